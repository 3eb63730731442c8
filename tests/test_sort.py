"""hfusion.sort (catalog module sort_ops): the oracle's literal restatement of
the reference's bubble-sort decomposition, pinned on the CPU against a
textbook stable sort (rows without NaN), against the closed form of where
the bubble passes leave NaNs (rows with NaN), and against hand-worked
answers on the shapes of the reference's own sort test; then the HIP
bitonic kernel against the oracle, bit-exact (GPU)."""
import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from helpers import run_gpu, run_oracle
from oracle import interp
from test_fusion import outline

SPEC = {s[0]: s for s in cat.SORT_OPS}
FLOATS = ("f32", "f16", "bf16")


def note(msg):
    print(f"[case] {msg}", flush=True)


def _nan_bits(elem, rng, n):
    """n NaNs of the element type with random payloads and signs (raw bits)."""
    if elem == "f32":
        return (0x7F800000 | rng.integers(1, 1 << 23, n) | (rng.integers(0, 2, n) << 31)).astype(np.uint32)
    if elem == "f16":
        return (0x7C00 | rng.integers(1, 1 << 10, n) | (rng.integers(0, 2, n) << 15)).astype(np.uint16)
    return (0x7F80 | rng.integers(1, 1 << 7, n) | (rng.integers(0, 2, n) << 15)).astype(np.uint16)


def values(elem, shape, rng, nan_rate=0.05):
    """Seeded values with many duplicates, +0 and -0, infinities and NaNs of
    several payloads (floats), or the integer extremes."""
    n = int(np.prod(shape))
    if elem in FLOATS:
        v = rng.choice(np.array([0.0, -0.0, 1.0, -1.0, 2.5, np.inf, -np.inf, 1e-3, -7.0], np.float32), n)
        v = np.where(rng.random(n) < 0.5, rng.normal(0, 10, n).astype(np.float32), v)
        if elem == "f32":
            bits = v.view(np.uint32).copy()
        else:
            import torch
            t = torch.from_numpy(v).to(torch.bfloat16 if elem == "bf16" else torch.float16)
            bits = t.view(torch.int16).numpy().view(np.uint16).copy()
        nan = rng.random(n) < nan_rate
        bits[nan] = _nan_bits(elem, rng, int(nan.sum()))
        return bits.reshape(shape) if elem != "f32" else bits.view(np.float32).reshape(shape)
    info = np.iinfo(interp.NP[elem])
    v = rng.integers(-20, 20, n)
    v = np.where(rng.random(n) < 0.05, rng.choice([info.min, info.max, 0, -1], n), v)
    return v.astype(interp.NP[elem]).reshape(shape)


def as_f32(a, elem):
    """Values of raw element storage, widened exactly to f32."""
    a = np.asarray(a)
    if elem == "f32":
        return a.astype(np.float32)
    if elem == "bf16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.view(np.float16).astype(np.float32)


def closed_form(x, elem, desc):
    """Where the bubble passes leave each element: NaNs (at index p) move to
    (p + 1) mod n with their bits, the other values are stably sorted into
    the remaining slots."""
    L = x.shape[-1]
    rows = np.asarray(x).reshape(-1, L)
    out = np.empty_like(rows)
    for r, row in enumerate(rows):
        f = as_f32(row, elem) if elem in FLOATS else row.astype(np.int64)
        nan = np.isnan(f) if elem in FLOATS else np.zeros(L, bool)
        idx = np.flatnonzero(~nan)
        keys = f[idx].astype(np.float64)
        order = idx[np.argsort(-keys if desc else keys, kind="stable")]
        slot_nan = np.roll(nan, 1)
        out[r, slot_nan] = np.roll(row, 1)[slot_nan]
        out[r, ~slot_nan] = row[order]
    return out.reshape(x.shape)


def oracle_sort(x, elem, desc):
    shape = list(x.shape)
    X = cat._T(shape, elem)
    ir = f"""module {{
  func.func @s(%x: {X}) -> {X}
      {cat._ATTRS.format(kind='ANY_PB')} {{
    %r = hfusion.sort ins(%x : {X}) descending = {str(desc).lower()} sort_axis = {len(shape) - 1} -> {X}
    return %r : {X}
  }}
}}
"""
    return interp.run(ir, x)[0]


@pytest.mark.parametrize("elem", ["f32", "f16", "bf16", "i8", "i16", "i32"])
@pytest.mark.parametrize("desc", [False, True])
def test_oracle_sort_is_stable_sort_without_nan(elem, desc):
    # a textbook stable sort of the values; +0 and -0 compare equal and keep
    # their input order, which a bit-level compare would catch
    rng = np.random.default_rng(11 + desc)
    x = values(elem, (7, 65), rng, nan_rate=0.0)
    got = oracle_sort(x, elem, desc)
    for r in range(x.shape[0]):
        f = as_f32(x[r], elem).astype(np.float64) if elem in FLOATS else x[r].astype(np.int64)
        want = x[r][np.argsort(-f if desc else f, kind="stable")]
        assert np.array_equal(np.asarray(got[r]).view(np.uint8), np.asarray(want).view(np.uint8)), r


@pytest.mark.parametrize("elem", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("desc", [False, True])
def test_oracle_sort_nan_closed_form(elem, desc):
    rng = np.random.default_rng(23 + desc)
    for L, rate in ((2, 0.5), (3, 0.4), (9, 0.3), (40, 0.2), (257, 0.05), (33, 1.0)):
        x = values(elem, (6, L), rng, nan_rate=rate)
        got, want = oracle_sort(x, elem, desc), closed_form(x, elem, desc)
        assert np.array_equal(np.asarray(got).view(np.uint8), want.view(np.uint8)), (L, rate)


def test_oracle_sort_known_answers():
    """Hand-worked bubble passes on the shapes of the reference's sort test
    (bishengir/test/Dialect/HFusion/test_sort.mlir: 6 ascending, 4x4
    ascending, 2x3x4 descending)."""
    nan = np.float32("nan")
    x = np.array([3, 1, nan, 2, -0.0, 0.0], np.float32)
    # pass 0: [1,3,nan,2,-0,0] -> 3 passes the NaN -> [1,nan,2,-0,0,3] ...
    # the NaN that started at 2 ends at 3; -0 stays before +0
    got = oracle_sort(x, "f32", False)
    assert np.array_equal(got.view(np.uint32), np.array([-0.0, 0.0, 1, nan, 2, 3], np.float32).view(np.uint32))
    x = np.array([[4, 3, 2, 1], [nan, 1, 0, -1], [1, 1, 1, 1], [-5, nan, 7, nan]], np.float32)
    want = np.array([[1, 2, 3, 4], [-1, nan, 0, 1], [1, 1, 1, 1], [nan, -5, nan, 7]], np.float32)
    got = oracle_sort(x, "f32", False)
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4) % 5
    want = -np.sort(-x, axis=-1)
    assert np.array_equal(oracle_sort(x, "f32", True), want)


def test_sort_lowering_limits(tmp_path):
    def ir(t, extra="", res=None, axis=None):
        res = res or t
        return f"""module {{
  func.func @s(%x: {t}) -> {res}
      {cat._ATTRS.format(kind='ANY_PB')} {{
    %r = hfusion.sort ins(%x : {t}) descending = false sort_axis = {axis if axis is not None else 1} -> {res}
    return %r : {res}
  }}
}}
"""
    for text, msg in ((ir("tensor<4x8xi64>"), "sort of i64"), (ir("tensor<4x8xf32>", axis=0), "axis other than the last"),
                      (ir("tensor<2x16385xf32>"), "longer than 16384")):
        with pytest.raises(hf.CompileError, match=msg):
            hf.compile(text, options="emit=hip")


@pytest.mark.gpu
@pytest.mark.parametrize("name", [s[0] for s in cat.SORT_OPS])
def test_sort_gpu(gpu, name):
    _, elem, shape, desc = SPEC[name]
    note(f"{name} {elem} {shape} desc={desc}")
    rng = np.random.default_rng(sum(map(ord, name)))
    x = values(elem, tuple(shape), rng)
    got, = run_gpu("sort_ops", [x], gpu, func=name)
    want, = run_oracle("sort_ops", [x], func=name)
    assert np.array_equal(np.asarray(got).view(np.uint8), np.asarray(want).view(np.uint8))
    # the closed form the kernel implements, checked at full size as well
    assert np.array_equal(np.asarray(got).view(np.uint8), closed_form(x, elem, desc).view(np.uint8))


@pytest.mark.gpu
def test_sort_gpu_all_nan_and_sorted_rows(gpu):
    name = "sort_f32_asc"
    note(name + " all-NaN / sorted / reversed rows")
    rng = np.random.default_rng(5)
    x = values("f32", (64, 1000), rng)
    x[0] = np.float32("nan")
    x[1] = np.sort(rng.normal(0, 1, 1000)).astype(np.float32)
    x[2] = x[1][::-1]
    x[3] = 0.0
    x[3, ::2] = -0.0
    got, = run_gpu("sort_ops", [x], gpu, func=name)
    want, = run_oracle("sort_ops", [x], func=name)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_sort_program_outlined(tmp_path):
    """2 * sort(-x): the sort becomes a group of its own between the two
    elementwise groups, and the whole function on the oracle matches the
    closed form."""
    groups, progs, _ = outline(cat.get("prog_neg_sort_scale"), tmp_path)
    assert [ops for _, _, ops in groups] == [["elemwise_unary"], ["sort"], ["elemwise_binary"]]
    rng = np.random.default_rng(3)
    x = values("f32", (37, 300), rng)
    got, = run_oracle("prog_neg_sort_scale", [x])
    with np.errstate(invalid="ignore"):
        want = (closed_form((-x).astype(np.float32), "f32", True) * np.float32(2)).astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])


@pytest.mark.gpu
def test_sort_program_gpu(gpu):
    note("prog_neg_sort_scale")
    rng = np.random.default_rng(4)
    x = values("f32", (37, 300), rng)
    got, = run_gpu("prog_neg_sort_scale", [x], gpu)
    want, = run_oracle("prog_neg_sort_scale", [x])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
