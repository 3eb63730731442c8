"""ANY_PBR and rank-N reduction groups (catalog module any_pbr_ops and the
batched RMSNorm+quant group): the CPU oracle against independent numpy
restatements (CPU), then the HIP column / row programs against the oracle
(GPU, marker gpu).

Meaning pinned here: linalg.reduce folds each output element serially along
the reduced index from its init, in the CPU loop nest's order
(ConvertHIVMToUpstream.cpp:573-752 for the HIVM form; linalg-to-loops
otherwise); reduce_with_index follows its region (HFusionOps.cpp:1507-1653):
res = max/min(in, v), index taken when res OGT/OLT (sgt/slt) v."""
import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from helpers import bf16_ulp_diff, run_gpu, run_oracle

I = hf.inputs


def note(msg):
    print(f"[case] {msg}", flush=True)


def inputs(name, seed=0x414E59):
    rng = np.random.default_rng(seed + sum(map(ord, name)))
    if name == "sumsq_mid":
        return [rng.normal(0, 1, (8, 64, 100)).astype(np.float32), np.zeros((8, 100), np.float32)]
    if name == "softmax_d0":
        return [rng.normal(0, 2, (512, 1000)).astype(np.float32), np.zeros((512, 1000), np.uint16)]
    if name == "argmax_mid":
        x = rng.integers(-50, 50, (16, 300, 40)).astype(np.float32) / 4  # many ties
        x[0, :, 0] = -np.inf          # nothing beats the init: index 0
        x[1, 7, 1] = np.nan           # NaN: value NaN, index from the prefix
        x[2, 0, 2] = np.nan           # NaN first: index stays at the init
        x[3, :, 3] = 0.0
        x[3, 9, 3] = -0.0             # +0 / -0 one class: the first wins
        x[4, 299, 4] = 1e30           # maximum in the last position
        return [x, np.zeros((16, 40), np.float32), np.zeros((16, 40), np.int32)]
    if name == "argmin_d0_i32":
        x = rng.integers(-20, 20, (1000, 64)).astype(np.int32)
        x[:, 5] = 2147483647          # never below the init: index 0
        x[500, 6] = -2147483648
        return [x, np.zeros(64, np.int32), np.zeros(64, np.int64)]
    if name == "argmax_fused":
        x = rng.normal(0, 1, (64, 777)).astype(np.float32)
        x[3, 100] = x[3].min()        # a tie of the maximum of -x
        x[5, 10] = np.nan
        return [x, np.zeros(64, np.float32), np.zeros(64, np.int32)]
    if name == "sum_rank3_last":
        x = rng.normal(0, 1, (8, 64, 100)).astype(np.float32)
        x[0, 0, 50:] = -x[0, 0, :50]         # a row that cancels
        x[1, 3, 50:] = -x[1, 3, :50] * 1.001  # a row that nearly cancels
        x[2, 5, :] = 1e-3
        x[2, 5, 0] = 3e4                      # absorbed small terms (order matters)
        return [x, np.zeros((8, 64), np.float32)]
    if name == "max_bias_rank3":
        x = rng.normal(0, 1, (4, 16, 256)).astype(np.float32)
        x[1, 2, 30] = np.nan
        return [x, rng.normal(0, 1, (16, 256)).astype(np.float32), np.zeros((4, 16), np.float32)]
    if name == "isum_d01":
        return [rng.integers(-2**31, 2**31, (6, 50, 33)).astype(np.int32), np.zeros(33, np.int32)]
    raise KeyError(name)


def serial_argfold(x, axis, init_v, init_i, kind):
    """The region folded literally, one reduced index at a time (vectorised
    over the kept points)."""
    xs = np.moveaxis(x, axis, 0)
    v = np.full(xs.shape[1:], init_v, x.dtype)
    i = np.full(xs.shape[1:], init_i, np.int64)
    for r in range(xs.shape[0]):
        xr = xs[r]
        if x.dtype == np.float32:
            with np.errstate(invalid="ignore"):
                res = np.where(np.isnan(xr) | np.isnan(v), np.float32(np.nan),
                               np.maximum(xr, v) if kind == "max" else np.minimum(xr, v)).astype(np.float32)
                upd = res > v if kind == "max" else res < v
        else:
            res = np.maximum(xr, v) if kind == "max" else np.minimum(xr, v)
            upd = res > v if kind == "max" else res < v
        i = np.where(upd, r, i)
        v = res
    return v, i


# ----------------------------------------------------------------- oracle (CPU)
def test_oracle_sumsq_mid_is_serial():
    x, o = inputs("sumsq_mid")
    ref, = run_oracle("any_pbr_ops", [x, o], func="sumsq_mid")
    acc = np.zeros((8, 100), np.float32)
    for r in range(64):  # serial along the reduced axis, f32 rounding per step
        acc = (acc + (x[:, r, :] * x[:, r, :]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(ref, (acc * np.float32(0.5)).astype(np.float32))


def test_oracle_softmax_d0_close_to_float64():
    x, o = inputs("softmax_d0")
    ref, = run_oracle("any_pbr_ops", [x, o], func="softmax_d0")
    e = np.exp(x.astype(np.float64) - x.max(axis=0))
    want = e / e.sum(axis=0)
    got = (ref.astype(np.uint32) << 16).view(np.float32)
    assert np.allclose(got, want, rtol=2 ** -7, atol=0)


@pytest.mark.parametrize("name,axis,kind,init_v", [("argmax_mid", 1, "max", -np.inf),
                                                   ("argmin_d0_i32", 0, "min", 2147483647)])
def test_oracle_reduce_with_index_region(name, axis, kind, init_v):
    args = inputs(name)
    v, i = run_oracle("any_pbr_ops", args, func=name)
    ev, ei = serial_argfold(args[0], axis, init_v, 0, kind)
    assert np.array_equal(i, ei)
    assert np.array_equal(np.isnan(v), np.isnan(ev)) if v.dtype == np.float32 else True
    ok = ~np.isnan(ev) if v.dtype == np.float32 else np.ones(v.shape, bool)
    assert np.array_equal(v[ok], ev[ok])
    if name == "argmax_mid":
        assert i[0, 0] == 0 and np.isnan(v[1, 1]) and i[2, 2] == 0 and i[3, 3] == 0 and i[4, 4] == 299


def test_oracle_sum_rank3_last_is_serial():
    x, o = inputs("sum_rank3_last")
    ref, = run_oracle("any_pbr_ops", [x, o], func="sum_rank3_last")
    acc = np.zeros((8, 64), np.float32)
    for c in range(100):
        acc = (acc + x[:, :, c]).astype(np.float32)
    assert np.array_equal(ref.view(np.uint32), acc.view(np.uint32))
    assert abs(ref[0, 0]) < 1e-4 * np.abs(x[0, 0]).sum()  # the cancelling row


def test_oracle_isum_d01_wraps():
    x, o = inputs("isum_d01")
    ref, = run_oracle("any_pbr_ops", [x, o], func="isum_d01")
    want = (x.astype(np.int64).reshape(300, 33).sum(axis=0) + 2**31) % 2**32 - 2**31
    assert np.array_equal(ref, want.astype(np.int32))


def test_oracle_max_bias_rank3():
    x, b, o = inputs("max_bias_rank3")
    ref, = run_oracle("any_pbr_ops", [x, b, o], func="max_bias_rank3")
    a = x + b[None]
    want = np.where(np.isnan(a).any(axis=2), np.float32(np.nan), np.nanmax(a, axis=2))
    assert np.array_equal(np.isnan(ref), np.isnan(want))
    assert np.array_equal(ref[~np.isnan(ref)], want[~np.isnan(want)])


def test_lowering_kinds(tmp_path):
    art = hf.compile(cat.get("any_pbr_ops"))
    kinds = {b["func"]: (b["kind"], b.get("variant", "")) for b in art.blocks}
    assert kinds["sumsq_mid"][0] == "ANY_PBR" and "dim 1 of 3" in kinds["sumsq_mid"][1]
    assert kinds["isum_d01"][0] == "ANY_PBR" and "dim 0 of 2" in kinds["isum_d01"][1]  # [6,50] collapse
    assert kinds["sum_rank3_last"][0] == "LAST_AXIS_PBR"  # rank 3 -> rows x 100
    assert "serial-order" in kinds["sum_rank3_last"][1]
    assert kinds["max_bias_rank3"][0] == "ANY_PBR"        # [S,C] operand: no row layout
    rq = hf.compile(cat.get("rmsnorm_quant_rank3")).blocks[0]
    assert rq["kind"] == "LAST_AXIS_PBR" and "binade-run exact serial sum" in rq.get("variant", "")


# ----------------------------------------------------------------- GPU parity
EXACT = ["sumsq_mid", "argmax_mid", "argmin_d0_i32", "argmax_fused", "max_bias_rank3", "isum_d01"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", EXACT)
def test_gpu_exact(gpu, name):
    note(f"any_pbr_ops {name}")
    args = inputs(name)
    outs = run_gpu("any_pbr_ops", args, gpu, func=name)
    refs = run_oracle("any_pbr_ops", args, func=name)
    for o, r in zip(outs, refs):
        assert o.dtype == r.dtype and o.shape == r.shape
        if o.dtype == np.float32:  # NaN payloads are not pinned: NaN positions must agree
            assert np.array_equal(np.isnan(o), np.isnan(r)), f"{name}: NaN positions differ"
            o, r = o[~np.isnan(r)], r[~np.isnan(r)]
        assert np.array_equal(np.asarray(o).view(np.uint8), np.asarray(r).view(np.uint8)), f"{name}: differs"


@pytest.mark.gpu
def test_gpu_softmax_d0(gpu):
    note("any_pbr_ops softmax_d0")
    args = inputs("softmax_d0")
    out, = run_gpu("any_pbr_ops", args, gpu, func="softmax_d0")
    ref, = run_oracle("any_pbr_ops", args, func="softmax_d0")
    assert bf16_ulp_diff(out, ref).max() <= 1


@pytest.mark.gpu
def test_gpu_sum_rank3_last(gpu):
    """Row sums of 100 elements fold in the reference's serial order on the
    GPU too (rows of up to 4096 elements take the serial schedule), so the
    fp32 results are bit-exact, cancelling rows included."""
    note("any_pbr_ops sum_rank3_last")
    args = inputs("sum_rank3_last")
    out, = run_gpu("any_pbr_ops", args, gpu, func="sum_rank3_last")
    ref, = run_oracle("any_pbr_ops", args, func="sum_rank3_last")
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.gpu
def test_gpu_rmsnorm_quant_rank3(gpu):
    """RMSNorm + dynamic int8 quant over [4, 64, 1024]: the rank-3 group
    collapses to 256 rows; codes and scales bit-exact."""
    note("rmsnorm_quant_rank3")
    x, g = I.config_inputs("rmsnorm_quant", rows=256, cols=1024)
    x = x.reshape(4, 64, 1024)
    args = [x, g, np.zeros((4, 64, 1024), np.int8), np.zeros((4, 64), np.float32)]
    q, s = run_gpu("rmsnorm_quant_rank3", args, gpu)
    rq, rs = run_oracle("rmsnorm_quant_rank3", args)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(q, rq)
