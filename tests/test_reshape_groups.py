"""Reshapes and transposes inside groups that reduce or broadcast.

The reference admits tensor.collapse_shape / expand_shape and
linalg.transpose into LAST_AXIS_PBR, ANY_PBR and ANY_PB groups
(bishengir/lib/Dialect/HFusion/Transforms/OpFusion/FusibleHelper.cpp:617-629),
and its own model-derived group
bishengir/test/Dialect/HFusion/hfusion-pipeline.mlir:56-125 holds both kinds
of reshape around four row sums (catalog `sig_sums`).  CPU: the oracle
against independent numpy restatements, the lowering's choices and the
fusion front-end on un-fused host IR.  GPU (marker gpu): the kernels against
the oracle, bit-exact."""
import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from helpers import run_gpu, run_oracle


def note(msg):
    print(f"[case] {msg}", flush=True)


# ----------------------------------------------------- numpy bf16 arithmetic
def b2f(u):
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f2b(f):
    """f32 -> bf16 bits, round to nearest even (finite values)."""
    u = np.asarray(f, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_normal(rng, shape, scale=1.0):
    return f2b(rng.normal(0, scale, shape).astype(np.float32))


def serial_sum(x2d):
    """Row sums folded left to right from +0 in f32 (the CPU loop's order)."""
    acc = np.zeros(x2d.shape[0], np.float32)
    for j in range(x2d.shape[1]):
        acc = (acc + x2d[:, j]).astype(np.float32)
    return acc


def sig_inputs(b, s, h, w, seed=0x5349):
    rng = np.random.default_rng(seed + b * s)
    a0, a1 = bf16_normal(rng, (b, s, h, w)), bf16_normal(rng, (b, s, h, w))
    a2, a3 = bf16_normal(rng, (b, s, 1, 1)), bf16_normal(rng, (b, s, 1, 1))
    a4 = rng.normal(0, 1, (b, s, h, w)).astype(np.float32)
    return [a0, a1, a2, a3, a4]  # the six results are buffers of their own


def sig_numpy(a0, a1, a2, a3, a4):
    """hfusion-pipeline.mlir:56-125 restated op by op: every bf16 op in f32
    then rounded to bf16; exp in float64 rounded to f32 (glibc's expf rounds
    alike except within 0.01 f32 ulp of a bf16 midpoint); serial f32 sums."""
    B, S, H, W = a0.shape
    op = lambda f, *xs: f2b(f(*[b2f(x) for x in xs]))  # noqa: E731
    b2 = np.broadcast_to(a2.reshape(B, S, 1, 1), a0.shape)
    b3 = np.broadcast_to(a3.reshape(B, S, 1, 1), a0.shape)
    one = f2b(np.float32(1.0))
    z = op(np.add, op(np.multiply, a1, b2), op(np.multiply, b3, one))
    ex = f2b(np.exp(-b2f(z).astype(np.float64)).astype(np.float32))
    sig = op(lambda d: np.float32(1) / d, op(lambda e: e + np.float32(1), ex))
    s13 = op(np.subtract, one, op(np.multiply, sig, one))
    s16 = op(np.add, op(np.multiply, z, s13), op(np.multiply, one, one))
    s18 = op(np.multiply, a0, op(np.multiply, sig, s16))
    f21 = b2f(op(np.multiply, s18, b2))
    f22 = (f21 * a4).astype(np.float32)
    r0 = serial_sum(f22.reshape(B * S, H * W)).reshape(B, S)
    r1 = serial_sum(f21.reshape(B * S, H * W)).reshape(B, S)
    r2 = serial_sum(b2f(op(np.multiply, s18, a1)).reshape(B * S, H * W)).reshape(B, S, 1, 1)
    r3 = serial_sum(b2f(s18).reshape(B * S, H * W)).reshape(B, S, 1, 1)
    return [r0, r1, r2, r3, f2b(r2), f2b(r3)]


@pytest.mark.parametrize("name,shape", [("sig_sums_small", (3, 40, 4, 6)), ("sig_sums", (24, 512, 16, 12))])
def test_oracle_sig_sums(name, shape):
    args = sig_inputs(*shape)
    got = run_oracle(name, args)
    want = sig_numpy(*args)
    for g, w in zip(got, want):
        assert g.shape == w.shape and g.dtype == w.dtype
        assert np.array_equal(g.view(np.uint8), w.view(np.uint8))


def rs_tr_inputs(name, seed=0x52535452):
    rng = np.random.default_rng(seed + sum(map(ord, name)))
    if name == "rs_bcast_pb":
        return [rng.normal(0, 1, (16, 8, 64)).astype(np.float32), rng.normal(0, 1, (16, 1, 1)).astype(np.float32),
                np.zeros((16, 8, 64), np.float32)]
    if name == "rs_sum_mid":
        return [rng.normal(0, 1, (6, 10, 20, 30)).astype(np.float32), np.zeros((6, 1, 30), np.float32)]
    if name == "tr_mul_sum":
        x = rng.normal(0, 1, (300, 64)).astype(np.float32)
        y = rng.normal(0, 1, (64, 300)).astype(np.float32)
        y[5] = x[:, 5]          # a row whose products are all positive
        y[6] = -x[:, 6]
        y[7, :150] = x[:150, 7]  # a cancelling row
        y[7, 150:] = -x[150:, 7]
        return [x, y, np.zeros(64, np.float32)]
    if name == "tr_argmax":
        x = f2b(rng.integers(-40, 40, (500, 40)).astype(np.float32) / 8)  # many ties
        x[:, 3] = 0xFF80       # all -inf: nothing beats the init, index 0
        x[17, 4] = 0x7FC0      # NaN
        x[:, 5] = 0x8000       # -0 everywhere ...
        x[250, 5] = 0x0000     # ... one +0: the first wins, IEEE-equal
        return [x, np.zeros(40, np.uint16), np.zeros(40, np.int32)]
    if name == "tr3_max_bias":
        x = rng.normal(0, 1, (12, 40, 70)).astype(np.float32)
        x[3, 7, 9] = np.nan
        return [x, rng.normal(0, 1, 70).astype(np.float32), np.zeros((70, 40), np.float32)]
    if name == "tr_bcast_sub":
        return [rng.normal(0, 1, (64, 100)).astype(np.float32), rng.normal(0, 1, 64).astype(np.float32),
                np.zeros((100, 64), np.float32)]
    raise KeyError(name)


def rs_tr_numpy(name, args):
    if name == "rs_bcast_pb":
        x, b, _ = args
        return [((x.reshape(16, 512) * b.reshape(16, 1)).astype(np.float32).reshape(16, 8, 64) - x).astype(np.float32)]
    if name == "rs_sum_mid":
        x, _ = args
        sq = (x * x).astype(np.float32).reshape(6, 200, 30)
        acc = np.zeros((6, 30), np.float32)
        for r in range(200):
            acc = (acc + sq[:, r, :]).astype(np.float32)
        return [np.sqrt(acc).reshape(6, 1, 30)]
    if name == "tr_mul_sum":
        x, y, _ = args
        return [serial_sum((x.T * y).astype(np.float32))]
    if name == "tr_argmax":
        x = b2f(args[0]).T  # [40, 500]
        v = np.full(40, -np.inf, np.float32)
        i = np.zeros(40, np.int64)
        for r in range(500):  # the region, literally: max then OGT update
            xr = x[:, r]
            # arith.maximumf: NaN-propagating, +0 above -0
            mx = np.where(xr == v, np.where(np.signbit(xr), v, xr), np.maximum(xr, v))
            with np.errstate(invalid="ignore"):
                res = np.where(np.isnan(xr) | np.isnan(v), np.float32(np.nan), mx).astype(np.float32)
                i = np.where(res > v, r, i)
            v = res
        return [f2b(np.where(np.isnan(v), np.float32(0), v)) | np.where(np.isnan(v), 0x7FC0, 0).astype(np.uint16),
                i.astype(np.int32)]
    if name == "tr3_max_bias":
        x, b, _ = args
        a = (np.transpose(x, (2, 0, 1)) + b[:, None, None]).astype(np.float32)
        return [np.where(np.isnan(a).any(axis=1), np.float32(np.nan), np.nanmax(a, axis=1))]
    if name == "tr_bcast_sub":
        x, b, _ = args
        return [(x.T - b[None, :]).astype(np.float32)]
    raise KeyError(name)


def same(a, b):
    """Bitwise equal, NaNs compared by position only (payloads are not pinned)."""
    if a.dtype == np.float32:
        if not np.array_equal(np.isnan(a), np.isnan(b)):
            return False
        a, b = a[~np.isnan(a)], b[~np.isnan(b)]
    if a.dtype == np.uint16:
        na, nb = (a & 0x7FFF) > 0x7F80, (b & 0x7FFF) > 0x7F80
        if not np.array_equal(na, nb):
            return False
        a, b = a[~na], b[~nb]
    return np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


@pytest.mark.parametrize("name", cat.RS_TR_OPS)
def test_oracle_rs_tr(name):
    args = rs_tr_inputs(name)
    got = run_oracle("rs_tr_ops", args, func=name)
    want = rs_tr_numpy(name, args)
    for g, w in zip(got, want):
        assert g.shape == w.shape, name
        assert same(g, w), name


def test_oracle_host_programs():
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (8, 16, 32)).astype(np.float32)
    got, = run_oracle("prog_rs_exp_sum_log", [x, np.zeros((8, 1), np.float32)])
    e = np.exp(x.astype(np.float64)).astype(np.float32).reshape(8, 512)
    want = np.log(serial_sum(e).astype(np.float64)).astype(np.float32).reshape(8, 1)
    assert np.allclose(got, want, rtol=2e-7, atol=0)
    args = rs_tr_inputs("tr_mul_sum")
    got, = run_oracle("prog_tr_mul_sum", args)
    assert np.array_equal(got, rs_tr_numpy("tr_mul_sum", args)[0])


# ----------------------------------------------------------- lowering (CPU)
def test_lowering_choices():
    blk = hf.compile(cat.get("sig_sums")).blocks[0]
    assert blk["kind"] == "LAST_AXIS_PBR" and "serial-order" in blk.get("variant", "")
    kinds = {b["func"]: (b["kind"], b.get("variant", "")) for b in hf.compile(cat.get("rs_tr_ops")).blocks}
    assert kinds["rs_bcast_pb"][0] == "ANY_PB"
    assert kinds["rs_sum_mid"] == ("ANY_PBR", "column program, serial along dim 1 of 3")  # [6, 200, 30]
    assert kinds["tr_mul_sum"][0] == "ANY_PBR" and kinds["tr_argmax"][0] == "ANY_PBR"
    assert "LDS-staged transpose" in kinds["tr_bcast_sub"][1]


@pytest.mark.parametrize("name", ["prog_rs_exp_sum_log", "prog_tr_mul_sum"])
def test_host_ir_fuses_into_one_group(name):
    """Un-fused host IR with a reshape (resp. a transpose) before a row sum:
    the front-end forms one group and the lowering takes it."""
    art = hf.compile(cat.get(name))
    assert len(art.blocks) == 1


def test_reshape_that_splits_a_kept_dim_is_refused():
    """A reduced [8] expanded to [2, 4]: no full-size tensor has that split,
    so the group has no common domain; the compiler says so."""
    X = "tensor<8x12xf32>"
    ir = f"""module {{
  func.func @bad(%x: {X}, %o: tensor<2x4xf32>) -> tensor<2x4xf32>
      attributes {{hacc.entry, hfusion.fusion_kind = #hfusion.fusion_kind<LAST_AXIS_PBR>}} {{
    %z = arith.constant 0.000000e+00 : f32
    %e = tensor.empty() : tensor<8xf32>
    %i = linalg.fill ins(%z : f32) outs(%e : tensor<8xf32>) -> tensor<8xf32>
    %s = linalg.reduce {{arith.addf}} ins(%x : {X}) outs(%i : tensor<8xf32>) dimensions = [1]
    %y = tensor.expand_shape %s [[0, 1]] output_shape [2, 4] : tensor<8xf32> into tensor<2x4xf32>
    %r = hfusion.elemwise_unary {{fun = #hfusion.unary_fn<sqrt>}} ins(%y : tensor<2x4xf32>) outs(%o : tensor<2x4xf32>) -> tensor<2x4xf32>
    return %r : tensor<2x4xf32>
  }}
}}
"""
    with pytest.raises(hf.CompileError, match="reshape splits a dim"):
        hf.compile(ir)


# ---------------------------------------------------------------- GPU parity
@pytest.mark.gpu
@pytest.mark.parametrize("name,shape", [("sig_sums_small", (3, 40, 4, 6)), ("sig_sums", (24, 512, 16, 12))])
def test_gpu_sig_sums(gpu, name, shape):
    """The reference's model-derived group at its own shape: every output
    bit-exact against the oracle (serial-order sums, guarded bf16 exp)."""
    note(f"{name} {shape}")
    args = sig_inputs(*shape)
    outs = run_gpu(name, args, gpu)
    refs = run_oracle(name, args)
    for k, (o, r) in enumerate(zip(outs, refs)):
        assert o.shape == r.shape and o.dtype == r.dtype
        assert np.array_equal(o.view(np.uint8), r.view(np.uint8)), f"{name}: result {k} differs"


@pytest.mark.gpu
@pytest.mark.parametrize("name", cat.RS_TR_OPS)
def test_gpu_rs_tr(gpu, name):
    note(f"rs_tr_ops {name}")
    args = rs_tr_inputs(name)
    outs = run_gpu("rs_tr_ops", args, gpu, func=name)
    refs = run_oracle("rs_tr_ops", args, func=name)
    for o, r in zip(outs, refs):
        assert o.shape == r.shape and o.dtype == r.dtype
        assert same(o, r), f"{name}: differs"


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["prog_rs_exp_sum_log", "prog_tr_mul_sum"])
def test_gpu_host_programs(gpu, name):
    note(name)
    if name == "prog_rs_exp_sum_log":
        rng = np.random.default_rng(7)
        args = [rng.normal(0, 1, (8, 16, 32)).astype(np.float32), np.zeros((8, 1), np.float32)]
    else:
        args = rs_tr_inputs("tr_mul_sum")
    out, = run_gpu(name, args, gpu)
    ref, = run_oracle(name, args)
    if name == "prog_rs_exp_sum_log":
        # f32 exp (6.5e-6 relative on the GPU, glibc on the CPU) summed, then log
        assert np.allclose(out, ref, rtol=1e-5, atol=0)
    else:
        assert np.array_equal(out, ref)
