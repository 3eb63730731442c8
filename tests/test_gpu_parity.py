"""GPU parity: each group runs through the HIP kernel (libhfr) and through the
CPU oracle (oracle/interp.py) on the same seeded inputs.

Bars: bit-exact for integer, index, quantised and exactly-rounded outputs;
<= 1 bf16 ulp where the result passes through exp or a reordered fp32 sum
before the final bf16 rounding; fp32 outputs within 1e-5 relative (plus a
row-scaled absolute term for outputs produced by cancellation).
"""
import json
import os

import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from helpers import (MATH_EXACT, bf16_ulp_diff, fp_funcs, fp_inputs, fuzz_inputs, fuzz_row_inputs, gather_inputs,
                     generic_inputs,
                     math_funcs,
                     math_inputs,
                     misc_extra_inputs,
                     misc_inputs, run_gpu, run_oracle, scan_inputs)

pytestmark = pytest.mark.gpu
I = hf.inputs
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def note(msg):
    print(f"[case] {msg}", flush=True)


def zeros(shape, dt):
    return np.zeros(shape, dt)


# ------------------------------------------------------------------ vec_add
def test_vec_add_golden_i16(gpu):
    note("vec_add_i16 golden (VecAdd/main.cpp)")
    g = json.load(open(os.path.join(GOLDEN, "vecadd_i16.json")))
    a, b = np.array(g["a"], np.int16), np.array(g["b"], np.int16)
    out, = run_gpu("vec_add_i16", [a, b, zeros(16, np.int16)], gpu)
    assert out.tolist() == g["expect"]


@pytest.mark.parametrize("name,n", [("vec_add_1m", 1 << 20), ("vec_add_ragged", 1001)])
def test_vec_add(gpu, name, n):
    note(name)
    a, b = I.config_inputs("vec_add", n=n)
    out, = run_gpu(name, [a, b, zeros(n, np.float32)], gpu)
    ref, = run_oracle(name, [a, b, zeros(n, np.float32)])
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------------ rmsnorm + quant
@pytest.mark.parametrize("name,rows,cols", [("rmsnorm_quant_256", 256, 4096), ("rmsnorm_quant_ragged", 13, 1000),
                                            ("rmsnorm_quant_w2048", 96, 2048), ("rmsnorm_quant_w3072", 64, 3072)])
def test_rmsnorm_quant(gpu, name, rows, cols):
    note(name)
    x, gamma = I.config_inputs("rmsnorm_quant", rows=rows, cols=cols)
    args = [x, gamma, zeros((rows, cols), np.int8), zeros(rows, np.float32)]
    q, s = run_gpu(name, args, gpu)
    rq, rs = run_oracle(name, args)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32)), "per-row scale must be bit-exact"
    assert np.array_equal(q, rq), f"{int((q != rq).sum())} int8 codes differ"


# ------------------------------------------------------------------ softmax
@pytest.mark.parametrize("name,rows,cols", [("safe_softmax_64", 64, 32768), ("safe_softmax_ragged", 33, 1000)])
def test_safe_softmax(gpu, name, rows, cols):
    note(name)
    x, = I.config_inputs("safe_softmax", rows=rows, cols=cols)
    args = [x, zeros((rows, cols), np.uint16)]
    out, = run_gpu(name, args, gpu)
    ref, = run_oracle(name, args)
    d = bf16_ulp_diff(out, ref)
    assert d.max() <= 1, f"max {d.max()} bf16 ulp"


# ------------------------------------------------------------------ argmax
def argmax_special(rows, cols, seed):
    x = I.argmax_logits(seed, rows, cols, dup_every=1)
    if rows >= 8:
        x[1, :] = -np.inf                       # no element beats the init -> index 0
        x[2, :] = 0.0
        x[2, 5] = -0.0                          # +0/-0 are one class: first of them wins
        x[3, cols // 3] = np.nan                # NaN: value NaN, index from the prefix
        x[4, 0] = np.nan                        # NaN first: index stays at init
        x[5, :] = 7.0                           # all equal -> 0
        x[6, cols - 1] = 1e30                   # maximum in the last element
        x[7, cols // 2] = np.inf
        x[7, cols // 2 + 3] = np.inf
    return x


@pytest.mark.parametrize("name,rows,cols,it", [("argmax_16", 16, 152064, np.int32), ("argmax_ragged", 5, 1001, np.int32),
                                               ("argmax_i64", 8, 4096, np.int64), ("argmin_ragged", 9, 5001, np.int32),
                                               ("argmax_tall", 2048, 33797, np.int32)])
def test_argmax(gpu, name, rows, cols, it):
    note(name)
    x = argmax_special(rows, cols, I.SEED_BASE + 30)
    if name.startswith("argmin"):
        x = -x   # the same special rows, mirrored for <min> (init +inf)
    args = [x, zeros(rows, np.float32), zeros(rows, it)]
    v, i = run_gpu(name, args, gpu)
    rv, ri = run_oracle(name, args)
    assert np.array_equal(i, ri)
    assert np.array_equal(np.isnan(v), np.isnan(rv))
    ok = ~np.isnan(rv)
    assert np.array_equal(v[ok].view(np.uint32), rv[ok].view(np.uint32))


def test_argmax_repeat_launch(gpu):
    """The per-row arrival counters reset themselves: two launches agree."""
    note("argmax_16 repeated")
    x = argmax_special(16, 152064, I.SEED_BASE + 31)
    args = [x, zeros(16, np.float32), zeros(16, np.int32)]
    a = run_gpu("argmax_16", args, gpu)
    b = run_gpu("argmax_16", args, gpu)
    assert all(np.array_equal(p, q, equal_nan=True) for p, q in zip(a, b))


# ------------------------------------------------------------------ W8A8
@pytest.mark.parametrize("name,m,n,k", [("w8a8_512", 512, 512, 512), ("w8a8_ragged", 300, 200, 160),
                                        ("w8a8_ragged_dma", 300, 200, 192), ("w8a8_ragged_dma128", 300, 200, 384),
                                        ("w8a8_kn", 320, 256, 128), ("w8a8_kn_ragged", 300, 208, 384),
                                        ("w8a8_kn_wide", 264, 784, 256), ("w8a8_kn_dma64", 300, 208, 192),
                                        ("w8a8_kn_tiny", 1, 16, 128)])
def test_w8a8(gpu, name, m, n, k):
    note(name)
    a, b, st, sc = I.config_inputs("w8a8_dequant", m=m, n=n, k=k)
    if "_kn" in name:
        b = np.ascontiguousarray(b.T)   # the same weights in the [K, N] layout
    args = [a, b, st, sc, zeros((m, n), np.uint16)]
    out, = run_gpu(name, args, gpu)
    ref, = run_oracle(name, args)
    assert np.array_equal(out, ref), f"max {bf16_ulp_diff(out, ref).max()} ulp"


def test_mm_i8_ragged(gpu):
    """int8 contraction with no epilogue: the raw int32 accumulator, exact."""
    note("mm_i8_ragged")
    s = I.SEED_BASE + 45
    a, b = I.int8_uniform(s, (300, 192)), I.int8_uniform(s + 1, (200, 192))
    c, = run_gpu("mm_i8_ragged", [a, b, zeros((300, 200), np.int32)], gpu)
    rc, = run_oracle("mm_i8_ragged", [a, b, zeros((300, 200), np.int32)])
    assert np.array_equal(c, rc)
    assert np.array_equal(c.astype(np.int64), a.astype(np.int64) @ b.astype(np.int64).T)


def _hivm_inputs(name):
    """Inputs of the hivm.hir.matmul catalog cases, argument order A, B,
    [bias], [descale], C."""
    s = I.SEED_BASE + 48
    f16 = lambda a: np.asarray(a, np.float16).view(np.uint16)
    if name == "hivm_mm_f16_at_bt":
        return [f16(I.normal_f32(s, (192, 152))), f16(I.normal_f32(s + 1, (264, 192))), np.zeros((152, 264), np.uint16)]
    if name.startswith("hivm_mm_f16"):
        a, b = I.normal_f32(s, (16, 16)), I.normal_f32(s + 1, (16, 16))
        args = [f16(a), f16(b)]
        if name != "hivm_mm_f16_null":
            args.append(f16(I.normal_f32(s + 2, (16,))))
            args.append(f16(I.uniform_f32(s + 3, (16 if name.endswith("_pc") else 1,), 0.5, 2.0)))
        return args + [np.zeros((16, 16), np.uint16)]
    if name == "hivm_mm_i8_pc":
        return [I.int8_uniform(s, (300, 192)), I.int8_uniform(s + 1, (200, 192)),
                (I.splitmix64(s + 2, 200) % np.uint64(2001)).astype(np.int32) - 1000,
                I.uniform_f32(s + 3, (200,), 0.001, 0.02), np.zeros((300, 200), np.uint16)]
    if name == "hivm_mm_i8_pt_i8out":
        return [I.int8_uniform(s, (256, 128)), I.int8_uniform(s + 1, (320, 128)), np.array([2e-3], np.float32),
                np.zeros((256, 320), np.int8)]
    if name in ("hivm_mm_i8_at", "hivm_mm_i8_at_kn"):
        m, n, k = (272, 320, 256) if name == "hivm_mm_i8_at" else (256, 208, 384)
        bshape = (n, k) if name == "hivm_mm_i8_at" else (k, n)
        ds = I.uniform_f32(s + 3, (n,) if name == "hivm_mm_i8_at" else (1,), 0.001, 0.02)
        return [I.int8_uniform(s, (k, m)), I.int8_uniform(s + 1, bshape), ds, np.zeros((m, n), np.uint16)]
    if name == "hivm_mm_bf16_at_bt":
        return [I.normal_bf16(s, (128, 200)), I.normal_bf16(s + 1, (136, 128)), np.zeros((200, 136), np.float32)]
    if name == "hivm_mm_bf16_at":
        return [I.normal_bf16(s, (64, 160)), I.normal_bf16(s + 1, (64, 96)), I.normal_f32(s + 2, (96,)),
                np.zeros((160, 96), np.float32)]
    raise KeyError(name)


@pytest.mark.parametrize("name", ["hivm_mm_f16_null", "hivm_mm_f16_bias_pc", "hivm_mm_f16_bias_pt_t", "hivm_mm_i8_pc",
                                  "hivm_mm_i8_pt_i8out", "hivm_mm_bf16_at", "hivm_mm_i8_at", "hivm_mm_i8_at_kn",
                                  "hivm_mm_bf16_at_bt", "hivm_mm_f16_at_bt"])
def test_hivm_matmul(gpu, name):
    """hivm.hir.matmul with bias / descale modes / transposes (written in place
    into the `outs` memref argument)."""
    note(name)
    args = _hivm_inputs(name)
    out, = run_gpu(name, args, gpu)
    ref, = run_oracle(name, args)
    if name.startswith("hivm_mm_i8"):
        assert np.array_equal(out, ref)               # exact int32 accumulator, same fp32 epilogue
    elif name == "hivm_mm_f16_at_bt":
        # 192-term sums: where they cancel, the f32 order difference (<= K * 2^-24 * sum|ab|)
        # can exceed an f16 ulp
        fa = args[0].view(np.float16).astype(np.float64).T
        fb = args[1].view(np.float16).astype(np.float64).T
        mag = np.abs(fa) @ np.abs(fb)
        o, r = out.view(np.float16).astype(np.float64), ref.view(np.float16).astype(np.float64)
        assert np.all(np.abs(o - r) <= 192 * 2.0 ** -24 * mag + 2.0 ** -10 * np.abs(r) + 2.0 ** -24)
    elif name.startswith("hivm_mm_f16"):
        assert bf16_ulp_diff(out, ref).max() <= 1      # f16 bits; fp32 sums in another order
    else:
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("name,m,n,k", [("bf16_mmad_256", 256, 256, 256), ("bf16_mmad_ragged", 200, 136, 96),
                                        ("bf16_mmad_ragged128", 200, 136, 192)])
def test_bf16_mmad(gpu, name, m, n, k):
    note(name)
    s = I.SEED_BASE + 40
    a, b = I.normal_bf16(s, (m, k)), I.normal_bf16(s + 1, (n, k))
    args = [a, b, zeros((m, n), np.uint16)]
    out, = run_gpu(name, args, gpu)
    ref, = run_oracle(name, args)
    # fp32 accumulation order differs from the serial k loop
    assert bf16_ulp_diff(out, ref).max() <= 1


@pytest.mark.parametrize("name,m,n,k,elem", [("bf16_mmad_kn", 256, 256, 128, "bf16"),
                                             ("bf16_mmad_kn_ragged", 200, 136, 192, "bf16"),
                                             ("f16_mmad_kn", 264, 520, 320, "f16"),
                                             ("bf16_mmad_kn_tiny", 3, 8, 64, "bf16")])
def test_mmad_16bit_kn(gpu, name, m, n, k, elem):
    """B [K, N] (linalg.matmul) in bf16 and f16: the ring stages whole k-rows
    and forms the operand with 16-bit transposing LDS reads."""
    note(name)
    s = I.SEED_BASE + 41
    if elem == "bf16":
        a, b = I.normal_bf16(s, (m, k)), I.normal_bf16(s + 1, (k, n))
    else:
        a = I.normal_f32(s, (m, k)).astype(np.float16).view(np.uint16)
        b = I.normal_f32(s + 1, (k, n)).astype(np.float16).view(np.uint16)
    args = [a, b, zeros((m, n), np.uint16)]
    out, = run_gpu(name, args, gpu)
    ref, = run_oracle(name, args)
    if elem == "bf16":
        # fp32 accumulation order differs from the serial k loop
        assert bf16_ulp_diff(out, ref).max() <= 1
    else:
        # f16 keeps 11 bits: where a 320-term sum cancels, the f32 order
        # difference (<= K * 2^-24 * sum|ab|) can exceed one f16 ulp, so the
        # bar is that plus half an ulp of each rounding
        fa, fb = (x.view(np.float16).astype(np.float64) for x in (a, b))
        mag = np.abs(fa) @ np.abs(fb)
        o, r = out.view(np.float16).astype(np.float64), ref.view(np.float16).astype(np.float64)
        assert np.all(np.abs(o - r) <= k * 2.0 ** -24 * mag + 2.0 ** -10 * np.abs(r) + 2.0 ** -24)


# ------------------------------------------------------------------ casts
def cast_inputs(n):
    v = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, 126.5, 127.5, -127.5, -128.5, 128.7, 127.5, 100.3, -129.2,
         -128.4, 300.7, -300.2, 1e-40, -1e-40, -0.0, 0.0, 3.0000002, 1.00390625, 1.0048828, 65504.0, 65520.0, 1e5,
         -1e5, 5.9604645e-08, 2.9802322e-08, 8.940697e-08]
    rnd = I.normal_f32(I.SEED_BASE + 50, (n,), std=200.0)
    x = np.concatenate([np.array(v, np.float32), rnd])[:n]
    return np.ascontiguousarray(x.astype(np.float32))


CAST_FUNCS = [f"cast_{t}_{m}{s}" for m in ["rint", "round", "floor", "ceil", "trunc", "odd"]
              for t, s in (("i8", "_sat"), ("i8", ""), ("i32", ""), ("bf16", ""), ("f16", ""))]


@pytest.mark.parametrize("func", CAST_FUNCS)
def test_cast_round_modes(gpu, func):
    note(func)
    n = 4096
    x = cast_inputs(n)
    tgt = func.split("_")[1]
    dt = {"i8": np.int8, "i32": np.int32, "bf16": np.uint16, "f16": np.uint16}[tgt]
    out, = run_gpu("cast_modes", [x, zeros(n, dt)], gpu, func=func)
    ref, = run_oracle("cast_modes", [x, zeros(n, dt)], func=func)
    assert np.array_equal(out, ref), f"{int((out != ref).sum())} differ, e.g. x={x[out != ref][:4]}"


@pytest.mark.parametrize("mode", ["rint", "round", "floor", "ceil", "trunc", "odd"])
def test_cast_int_and_same_type(gpu, mode):
    note(f"cast i32->f32 / f32->f32 {mode}")
    n = 4096
    xi = np.concatenate([np.array([16777217, -16777217, 16777219, 2147483647, -2147483648, 33554435, 7, -7], np.int32),
                         (I.splitmix64(I.SEED_BASE + 51, n - 8) >> np.uint64(32)).astype(np.uint32).view(np.int32)])
    out, = run_gpu("cast_modes", [xi, zeros(n, np.float32)], gpu, func=f"cast_i32_f32_{mode}")
    ref, = run_oracle("cast_modes", [xi, zeros(n, np.float32)], func=f"cast_i32_f32_{mode}")
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    x = cast_inputs(n)
    out, = run_gpu("cast_modes", [x, zeros(n, np.float32)], gpu, func=f"cast_f32_f32_{mode}")
    ref, = run_oracle("cast_modes", [x, zeros(n, np.float32)], func=f"cast_f32_f32_{mode}")
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------------ fp8
def fp8_cast_inputs(n, maxf, seed):
    """Values across the fp8 range: random, ties of the grid, subnormals,
    the overflow boundaries, signed zeros, inf and NaN."""
    r = I.normal_f32(seed, (n - 64,), std=maxf / 8)
    sp = np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, maxf, -maxf, maxf * 1.03, maxf * 1.04, maxf * 1.0714, maxf * 1.2,
                     -maxf * 1.2, 1e-9, -1e-9, 2.0 ** -9, 1.5 * 2.0 ** -9, 2.0 ** -16, 2.5 * 2.0 ** -16, 0.5625, 0.59375,
                     1.0625, 1.1875, 3.25, 13.0, 17.0, 52.0, 416.0, 432.0, 464.0, 240.0, 3e4, 6e4])
    return np.concatenate([sp, np.resize(sp, 64 - sp.size), r]).astype(np.float32)


FP8_FUNCS = [f"cast_{t}_{m}{s}" for t in ("e4m3", "e5m2") for m in ("rint", "round", "floor", "ceil", "trunc", "odd")
             for s in ("", "_sat")]


@pytest.mark.parametrize("func", FP8_FUNCS)
def test_cast_fp8(gpu, func):
    note(func)
    n = 4096
    maxf = 448.0 if "e4m3" in func else 57344.0
    x = fp8_cast_inputs(n, maxf, I.SEED_BASE + 80)
    out, = run_gpu("cast_fp8", [x, zeros(n, np.uint8)], gpu, func=func)
    ref, = run_oracle("cast_fp8", [x, zeros(n, np.uint8)], func=func)
    assert np.array_equal(out, ref), f"{int((out != ref).sum())} differ, e.g. x={x[out != ref][:4]}"


@pytest.mark.parametrize("func", ["dec_e4m3", "dec_e5m2", "f16_to_e5m2", "e5m2_to_f16", "ovf_i16_trunc", "ovf_i8_trunc"])
def test_cast_fp8_decode_and_marks(gpu, func):
    note(func)
    n = 4096
    if func.startswith("dec_") or func == "e5m2_to_f16":
        x = np.resize(np.arange(256, dtype=np.uint8), n)
    elif func == "f16_to_e5m2":
        x = fp8_cast_inputs(n, 57344.0, I.SEED_BASE + 81).astype(np.float16).view(np.uint16)
    else:
        x = I.normal_f32(I.SEED_BASE + 82, (n,), std=3e4 if "i16" in func else 300.0)
    o_dt = {"dec": np.float32, "f16_to_e5m2": np.uint8, "e5m2_to_f16": np.uint16, "ovf_i16_trunc": np.int16,
            "ovf_i8_trunc": np.int8}
    dt = o_dt["dec"] if func.startswith("dec_") else o_dt[func]
    out, = run_gpu("cast_fp8", [x, zeros(n, dt)], gpu, func=func)
    ref, = run_oracle("cast_fp8", [x, zeros(n, dt)], func=func)
    if dt == np.float32:
        assert np.array_equal(np.isnan(out), np.isnan(ref))
        ok = ~np.isnan(ref)
        assert np.array_equal(out[ok].view(np.uint32), ref[ok].view(np.uint32))
    elif func == "e5m2_to_f16":
        nan = (ref & 0x7C00) == 0x7C00
        assert np.array_equal(out[~nan | ((ref & 0x3FF) == 0)], ref[~nan | ((ref & 0x3FF) == 0)])
    else:
        assert np.array_equal(out, ref)
    if func.startswith("ovf_"):
        info = np.iinfo(dt)
        assert (out == info.max).any() and (out == info.min).any()  # saturation happened


@pytest.mark.parametrize("name,rows,cols", [("fp8_quant", 64, 4096), ("fp8_quant_ragged", 13, 1000)])
def test_fp8_quant(gpu, name, rows, cols):
    note(name)
    x = I.normal_bf16(I.SEED_BASE + 83, (rows, cols))
    args = [x, zeros((rows, cols), np.uint8), zeros(rows, np.float32)]
    q, s = run_gpu(name, args, gpu)
    rq, rs = run_oracle(name, args)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(q, rq), f"{int((q != rq).sum())} fp8 codes differ"


# ------------------------------------------------------------------ generic lowering
def test_eltwise_mix(gpu):
    note("eltwise_mix")
    s = I.SEED_BASE + 60
    x = I.normal_f32(s, (64, 1000))
    b = I.normal_f32(s + 1, (1000,))
    sc = I.uniform_f32(s + 2, (64,), 0.5, 2.0)
    args = [x, b, sc, zeros((64, 1000), np.uint16), zeros((64, 1000), np.bool_)]
    y, mask = run_gpu("eltwise_mix", args, gpu)
    ry, rmask = run_oracle("eltwise_mix", args)
    assert np.array_equal(mask, rmask)
    assert bf16_ulp_diff(y, ry).max() <= 1  # exp: GPU vs glibc expf


def test_layernorm(gpu):
    note("layernorm")
    s = I.SEED_BASE + 70
    x = I.normal_f32(s, (64, 2048), std=3.0) + np.float32(1.5)
    w, bias = I.uniform_f32(s + 1, (2048,), 0.5, 1.5), I.uniform_f32(s + 2, (2048,), -0.5, 0.5)
    args = [x, w, bias, zeros((64, 2048), np.float32), zeros(64, np.float32)]
    y, mu = run_gpu("layernorm", args, gpu)
    ry, rmu = run_oracle("layernorm", args)
    np.testing.assert_allclose(mu, rmu, rtol=1e-5, atol=1e-6)
    # tree vs serial sums: 1e-5 relative, absolute term scaled by the row's magnitude
    np.testing.assert_allclose(y, ry, rtol=1e-5, atol=1e-5 * np.abs(ry).max())


def test_reduce_ops(gpu):
    note("reduce_ops")
    s = I.SEED_BASE + 80
    x = I.normal_f32(s, (48, 3000))
    x[3, 17] = np.nan
    x[4, :] = -0.0
    x[4, 9] = 0.0
    xi = (I.splitmix64(s + 1, 48 * 3000) % np.uint64(2000001)).astype(np.int64).astype(np.int32).reshape(48, 3000) - 1000000
    args = [x, xi, zeros(48, np.float32), zeros(48, np.float32), zeros(48, np.float32), zeros(48, np.int32)]
    got = run_gpu("reduce_ops", args, gpu)
    ref = run_oracle("reduce_ops", args)
    for k, (g_, r_) in enumerate(zip(got, ref)):
        g_, r_ = np.asarray(g_), np.asarray(r_)
        if k < 3:
            assert np.array_equal(np.isnan(g_), np.isnan(r_))
            ok = ~np.isnan(r_)
            g_, r_ = g_[ok], r_[ok]
        if k == 2:
            # maxnumf leaves the sign of a zero maximum unspecified
            assert np.array_equal(g_, r_)
        else:
            assert np.array_equal(g_.view(np.uint32), r_.view(np.uint32))


def test_rint_of_row_division_near_ties(gpu):
    """nearbyint(x / s[row]): quotients on, and a few ulp around, half-integers,
    signed zeros, huge quotients (exact-path fallback) and specials."""
    note("quant_ties")
    rows, cols = 64, 1024
    s = I.uniform_f32(I.SEED_BASE + 90, (rows,), 0.001, 0.02)
    s[5] = 3.0e-39   # denormal divisor: reciprocal overflows
    s[6] = 1.0e-30   # huge quotients -> guarded exact path for this block
    k = (I.splitmix64(I.SEED_BASE + 91, rows * cols) % np.uint64(255)).astype(np.int64).reshape(rows, cols) - 127
    half = (k.astype(np.float64) + 0.5) * s[:, None].astype(np.float64)
    x = half.astype(np.float32)
    # nudge by -3..+3 ulp around the exact tie
    nud = ((I.splitmix64(I.SEED_BASE + 92, rows * cols) % np.uint64(7)).astype(np.int64) - 3).reshape(rows, cols)
    xb = x.view(np.int32) + nud.astype(np.int32)
    x = xb.view(np.float32).copy()
    x[0, :8] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3e38]
    x[1, :] = np.float32(0.5) * s[1]  # exact ties
    args = [x, s, np.zeros((rows, cols), np.float32), np.zeros(rows, np.float32)]
    out, mx = run_gpu("quant_ties", args, gpu)
    ref, rmx = run_oracle("quant_ties", args)
    assert np.array_equal(mx, rmx, equal_nan=True)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(out[ok].view(np.uint32), ref[ok].view(np.uint32)), int((out[ok] != ref[ok]).sum())


# ------------------------------------------------------ launch programs
# Un-fused host functions split by the fusion front-end into several groups;
# the whole program runs on the GPU (hfr_program_launch) and is compared with
# the oracle run over the un-fused function.
def _gemm_args(m, n, k):
    s = I.SEED_BASE + 70
    return [I.int8_uniform(s, (m, k)), I.int8_uniform(s + 1, (n, k)), I.uniform_bf16(s + 2, (n,), 0.5, 1.5),
            zeros((m, n), np.int8), zeros(m, np.float32)]


@pytest.mark.parametrize("name,shape", [("prog_gemm_rmsnorm_quant", (256, 512, 256)),
                                        ("prog_gemm_rmsnorm_quant_ragged", (100, 320, 192))])
def test_program_gemm_rmsnorm_quant(gpu, name, shape):
    """int8 contraction (exact) -> dequant -> RMSNorm -> int8 quant: every
    output bit-exact."""
    note(name)
    args = _gemm_args(*shape)
    q, sc = run_gpu(name, args, gpu)
    rq, rsc = run_oracle(name, args)
    assert np.array_equal(sc.view(np.uint32), rsc.view(np.uint32))
    assert np.array_equal(q, rq)


@pytest.mark.parametrize("name,shape", [("prog_scores_softmax", (128, 1024, 128)),
                                        ("prog_scores_softmax_ragged", (72, 1000, 64))])
def test_program_scores_softmax(gpu, name, shape):
    """bf16 contraction (fp32 accumulation order differs from the serial k
    loop) -> scale -> softmax -> bf16: within 1 bf16 ulp."""
    note(name)
    s = I.SEED_BASE + 80
    m, n, k = shape
    args = [I.normal_bf16(s, (m, k)), I.normal_bf16(s + 1, (n, k)), zeros((m, n), np.uint16)]
    out, = run_gpu(name, args, gpu)
    ref, = run_oracle(name, args)
    assert bf16_ulp_diff(out, ref).max() <= 1


@pytest.mark.parametrize("name,cols", [("quant_i8_ties", 1024), ("quant_i8_ties_m128", 1024),
                                       ("quant_i8_ties_narrow", 1000)])
def test_int8_quant_near_ties(gpu, name, cols):
    """(int8)clamp(nearbyint(x / s[row])) through the packed fast path:
    quotients on and a few ulp around half-integers (the bracketing check
    sends those blocks to the exact path), beyond the clamp bounds, specials."""
    note(name)
    rows = 64
    s = I.uniform_f32(I.SEED_BASE + 95, (rows,), 0.001, 0.02)
    s[5] = 3.0e-39   # denormal divisor: reciprocal overflows
    s[6] = 1.0e-30   # huge quotients
    k = (I.splitmix64(I.SEED_BASE + 96, rows * cols) % np.uint64(301)).astype(np.int64).reshape(rows, cols) - 150
    x = ((k.astype(np.float64) + 0.5) * s[:, None].astype(np.float64)).astype(np.float32)
    nud = ((I.splitmix64(I.SEED_BASE + 97, rows * cols) % np.uint64(7)).astype(np.int64) - 3).reshape(rows, cols)
    x = (x.view(np.int32) + nud.astype(np.int32)).view(np.float32).copy()
    # rows 10..39: quotients well inside the range and away from ties, so
    # those blocks stay on the fast path
    fr = (I.splitmix64(I.SEED_BASE + 98, 30 * cols) % np.uint64(1000)).astype(np.float64).reshape(30, cols) / 1000.0
    kk = k[10:40] % 200 - 100
    x[10:40] = ((kk + 0.05 + 0.4 * fr) * s[10:40, None].astype(np.float64)).astype(np.float32)
    x[0, :8] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3e38]
    x[1, :] = np.float32(0.5) * s[1]  # exact ties
    args = [x, s, np.zeros((rows, cols), np.int8), np.zeros(rows, np.float32)]
    out, mx = run_gpu(name, args, gpu)
    ref, rmx = run_oracle(name, args)
    assert np.array_equal(mx, rmx, equal_nan=True)
    assert np.array_equal(out, ref), int((out != ref).sum())


# ------------------------------------------------- elementwise function coverage
@pytest.mark.parametrize("func", math_funcs())
def test_math_fns(gpu, func):
    """Each elementwise function of the region builder on its domain and
    edges.  Integer functions, bitcast operands and the exactly rounded float
    functions are bit-exact; the transcendental ones (device libm against
    glibc) are within 1e-5 relative, with an absolute 1e-6 bar where the
    result crosses zero, and agree on NaN and infinity positions."""
    note(f"math_fns {func}")
    args = math_inputs(func)
    out, = run_gpu("math_fns", args, gpu, func=func)
    ref, = run_oracle("math_fns", args, func=func)
    if func in MATH_EXACT or func.startswith("i_"):
        assert np.array_equal(out.view(np.uint8), ref.view(np.uint8)) or np.array_equal(out, ref, equal_nan=True), \
            f"{int((out != ref).sum())} differ"
        return
    assert np.array_equal(np.isnan(out), np.isnan(ref)), "NaN positions differ"
    inf = np.isinf(ref) | np.isinf(out)
    assert np.array_equal(out[inf], ref[inf]), "infinities differ"
    fin = np.isfinite(ref) & np.isfinite(out)
    np.testing.assert_allclose(out[fin], ref[fin], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("func", fp_funcs())
def test_fp_ops(gpu, func):
    """HFusion float ops without outs and hfusion.bitcast: predicates,
    nextafter, hypot (the reference lowering's scaled f32 / direct f16
    algorithm) and bitcast are bit-exact; erfinv (double Newton on erf) and
    cyl_bessel_i0 (power series in double) within 1e-5 relative of the oracle's float64 erfinv, NaN/inf positions
    equal."""
    note(f"fp_ops {func}")
    args = fp_inputs(func)
    out, = run_gpu("fp_ops", args, gpu, func=func)
    ref, = run_oracle("fp_ops", args, func=func)
    if not func.startswith(("erfinv", "cylbesseli0")):
        same = out.view(np.uint8) == ref.view(np.uint8)
        if not same.all():
            # any NaN matches any NaN
            f = (lambda a: a.view(np.float16)) if func.endswith("f16") else (lambda a: a)
            a, b = f(out), f(ref)
            ok = (a == b) | (np.isnan(a.astype(np.float32)) & np.isnan(b.astype(np.float32)))
            assert ok.all(), f"{int((~ok).sum())} differ"
        return
    a = out.view(np.float16).astype(np.float32) if func.endswith("f16") else out
    b = ref.view(np.float16).astype(np.float32) if func.endswith("f16") else ref
    assert np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[np.isinf(b)], b[np.isinf(b)])
    fin = np.isfinite(b)
    np.testing.assert_allclose(a[fin], b[fin], rtol=1e-5 if func.endswith("f32") else 1e-3, atol=1e-7)


# ----------------------------------------- scans, histogram, (de)interleave
@pytest.mark.parametrize("name", [s[0] for s in cat.SCAN_OPS])
def test_scan_ops(gpu, name):
    """Cumulative ops in the serial order and per-step rounding of the CPU
    loop: bit-exact (NaN positions included)."""
    note(f"scan_ops {name}")
    args = scan_inputs(name)
    out, = run_gpu("scan_ops", args, gpu, func=name)
    ref, = run_oracle("scan_ops", args, func=name)
    if out.dtype.kind == "f":
        assert np.array_equal(out, ref, equal_nan=True), f"{int((out != ref).sum())} differ"
    else:
        assert np.array_equal(out, ref), f"{int((out != ref).sum())} differ"


@pytest.mark.parametrize("name", [h[0] for h in cat.HIST_OPS] + [i[0] for i in cat.INTERLEAVE_OPS])
def test_misc_ops(gpu, name):
    """histogram counts (twice in a row: the workspace is left cleared) and
    (de)interleave: bit-exact."""
    note(f"misc_ops {name}")
    args = misc_inputs(name)
    refs = run_oracle("misc_ops", args, func=name)
    for _ in range(2):
        outs = run_gpu("misc_ops", args, gpu, func=name)
        for o, r in zip(outs, refs):
            assert np.array_equal(o, r), f"{int((o != r).sum())} differ"


def test_program_with_scan(gpu):
    """Host function exp -> cumsum -> mul: three launches (the scan is a
    kernel of its own); exp on the GPU is within 6.5e-6 relative of glibc's,
    and the serial sum carries that, so 1e-5 relative (plus a row-scaled
    absolute term) bounds the result."""
    note("prog_exp_cumsum_scale")
    s = I.SEED_BASE + 90
    x = I.normal_f32(s, (64, 1000))
    w = I.uniform_f32(s + 1, (64, 1000), 0.5, 1.5)
    out, = run_gpu("prog_exp_cumsum_scale", [x, w], gpu)
    ref, = run_oracle("prog_exp_cumsum_scale", [x, w])
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())


@pytest.mark.parametrize("name", cat.MISC_EXTRA)
def test_flip_mulext_arange(gpu, name):
    """flip, mulext / mulextui (both halves) and arange (offset argument,
    negative stride, i32 and f32 results): bit-exact."""
    note(f"misc_ops {name}")
    args = misc_extra_inputs(name)
    outs = run_gpu("misc_ops", args, gpu, func=name)
    refs = run_oracle("misc_ops", args, func=name)
    assert len(outs) == len(refs)
    for o, r in zip(outs, refs):
        assert np.array_equal(o, r), f"{int((o != r).sum())} differ"


@pytest.mark.parametrize("name", [g[0] for g in cat.GATHER_OPS])
def test_gather(gpu, name):
    """hfusion.gather along axis 1 and 0 with out-of-range indices (init
    kept): bit-exact."""
    note(f"gather_ops {name}")
    args = gather_inputs(name)
    out, = run_gpu("gather_ops", args, gpu, func=name)
    ref, = run_oracle("gather_ops", args, func=name)
    assert np.array_equal(out, ref), f"{int((out != ref).sum())} differ"


def test_memref_chain(gpu):
    """Memref-form group: sqrt into %tmp, then %tmp + %x into %y; both written
    buffers come back, bit-exact."""
    note("memref_chain")
    x = np.abs(I.normal_f32(I.SEED_BASE + 95, (4096,)))
    args = [x, np.zeros(4096, np.float32), np.zeros(4096, np.float32)]
    outs = run_gpu("memref_chain", args, gpu)
    refs = run_oracle("memref_chain", args)
    assert len(outs) == 2 and len(refs) == 2
    for o, r in zip(outs, refs):
        assert np.array_equal(o, r)
    assert np.array_equal(refs[1], np.sqrt(x) + x)


def test_reshape_chain(gpu):
    """add -> expand_shape -> mul -> collapse_shape -> abs in one group: the
    reshapes are views of the flat index; bit-exact."""
    note("reshape_chain")
    s = I.SEED_BASE + 97
    args = [I.normal_f32(s, (128, 256)), I.normal_f32(s + 1, (128, 256)), I.normal_f32(s + 2, (32, 4, 256))]
    out, = run_gpu("reshape_chain", args, gpu)
    ref, = run_oracle("reshape_chain", args)
    assert np.array_equal(out, ref)
    assert np.array_equal(ref, np.abs(((args[0] + args[1]).reshape(32, 4, 256) * args[2]).reshape(128, 256)))


def test_generic_ops(gpu):
    """linalg.generic regions: the f16/int group bit-exact; the exp/tanh group
    (device exp and tanh against glibc) within 1e-5 relative."""
    note("generic_ops generic_bias_act")
    args = generic_inputs("generic_bias_act")
    out, = run_gpu("generic_ops", args, gpu, func="generic_bias_act")
    ref, = run_oracle("generic_ops", args, func="generic_bias_act")
    np.testing.assert_allclose(out, ref, rtol=1e-5)
    note("generic_ops generic_f16_int")
    args = generic_inputs("generic_f16_int")
    outs = run_gpu("generic_ops", args, gpu, func="generic_f16_int")
    refs = run_oracle("generic_ops", args, func="generic_f16_int")
    for o, r in zip(outs, refs):
        assert np.array_equal(o, r), f"{int((o != r).sum())} differ"


def test_rank0_group(gpu):
    """A group over rank-0 tensors runs as one element: bit-exact."""
    note("rank0")
    args = [np.array(2.5, np.float32), np.array(3.0, np.float32)]
    out, = run_gpu("rank0", args, gpu)
    ref, = run_oracle("rank0", args)
    assert np.array_equal(np.asarray(out).reshape(()), np.asarray(ref).reshape(()))
    assert float(np.asarray(ref)) == float(np.sqrt(np.float32(7.5)))


@pytest.mark.parametrize("n", range(12))
def test_fuzz_generic(gpu, n):
    """Seeded random linalg.generic regions of exactly rounded ops over f32 /
    f16 with a row-broadcast operand and an i32 operand: bit-exact (any NaN
    matches any NaN)."""
    note(f"fuzz_generic fuzz{n}")
    args, ft = fuzz_inputs(n)
    out, = run_gpu("fuzz_generic", args, gpu, func=f"fuzz{n}")
    ref, = run_oracle("fuzz_generic", args, func=f"fuzz{n}")
    a = out.view(np.float16).astype(np.float32) if ft == "f16" else out
    b = ref.view(np.float16).astype(np.float32) if ft == "f16" else ref
    same = (out == ref) | (np.isnan(a) & np.isnan(b))
    assert same.all(), f"{int((~same).sum())} differ, e.g. gpu={a[~same][:3]} oracle={b[~same][:3]}"


@pytest.mark.parametrize("n", range(8))
def test_fuzz_rows(gpu, n):
    """Seeded random row programs (elementwise chain -> max/min row reduce ->
    broadcast -> chain) over several row widths incl. ragged ones and 33000
    columns: bit-exact, NaN rows included."""
    note(f"fuzz_rows frow{n}")
    args = fuzz_row_inputs(n)
    outs = run_gpu("fuzz_rows", args, gpu, func=f"frow{n}")
    refs = run_oracle("fuzz_rows", args, func=f"frow{n}")
    for o, r in zip(outs, refs):
        same = (o == r) | (np.isnan(o) & np.isnan(r))
        assert same.all(), f"{int((~same).sum())} differ, e.g. gpu={o[~same][:3]} oracle={r[~same][:3]}"


def test_generic_reduce(gpu):
    """linalg.generic row reductions (split into an elementwise generic and a
    row reduction): max bit-exact; the float sum within 1e-5 relative plus a
    row-scaled absolute term (reduction order differs from the serial loop)."""
    note("generic_reduce")
    rng = np.random.default_rng(11)
    x = rng.normal(size=(64, 1000)).astype(np.float32)
    w = rng.normal(size=1000).astype(np.float32)
    args = [x, w, np.zeros(64, np.float32)]
    out, = run_gpu("generic_reduce", args, gpu, func="gred_max")
    ref, = run_oracle("generic_reduce", args, func="gred_max")
    assert np.array_equal(out, ref)
    out, = run_gpu("generic_reduce", args, gpu, func="gred_sum")
    ref, = run_oracle("generic_reduce", args, func="gred_sum")
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5 * np.abs(x * w).sum(axis=1).max())
