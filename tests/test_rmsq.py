"""The RMSNorm + dynamic int8 quantisation kernel (hf_rmsq.h, the default for
rows of 1024, 2048 or 4096 columns; option rmsq_kernel=0 selects
the generic row program, catalog names ending in _rowprog): its exact
serial fp32 sum of squares (binade runs composed across lanes, stitched from
the init) on rows built to stress every path of the stitch, bit-exact against
the CPU oracle's serial loop.

Rows (bf16, 4096 wide): N(0, s) at several scales (the binade of the running
sum crosses lane and sub-segment boundaries at different places), constants
(every step a tie or exact), exact powers of two, zeros, a NaN, an infinity,
squares that overflow, squares below the f32 normal range, and rows whose
sum crosses a binade exactly at a sub-segment boundary."""
import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from helpers import run_gpu, run_oracle

I = hf.inputs
C = 4096


def bf16(a):
    a = np.asarray(a, np.float32)
    b = a.view(np.uint32)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(a), np.uint16(0x7FC0), r)


def stress_rows(rows=256, seed=0x524D53):
    rng = np.random.default_rng(seed)
    x = np.zeros((rows, C), np.float32)
    for r in range(rows):
        kind = r % 16
        if kind < 6:
            x[r] = rng.normal(0, [1e-3, 0.1, 1, 3, 30, 1e4][kind], C)
        elif kind == 6:
            x[r] = 1.5                        # x^2 = 2.25: ties at every binade past 2^22 ulps
        elif kind == 7:
            x[r] = 2.0 ** rng.integers(-8, 8, C)
        elif kind == 8:
            x[r] = 0.0
            x[r, rng.integers(0, C)] = 1.0 if r % 32 == 8 else 0.0
        elif kind == 9:
            x[r] = rng.normal(0, 1, C)
            x[r, rng.integers(0, C)] = np.nan
        elif kind == 10:
            x[r] = rng.normal(0, 1, C)
            x[r, rng.integers(0, C)] = np.inf if r % 32 == 10 else -np.inf
        elif kind == 11:
            x[r] = rng.normal(0, 1e19, C)     # squares near the f32 maximum: the sum overflows
        elif kind == 12:
            x[r] = rng.normal(0, 1e-21, C)    # squares below 2^-126
        elif kind == 13:
            x[r] = 1.0                        # the sum reaches 2^k exactly at element 2^k
        elif kind == 14:
            x[r] = rng.choice([0.0, 1.0, 0.5, 0.25], C)
        else:
            x[r] = rng.normal(0, 1, C) * (rng.random(C) < 0.05)
    return bf16(x)


def fuzz_rows(rows=256, seed=0):
    """Rows of mixed shape, seeded: a scale 10^U(-25, 25) per row (and per
    segment of 64 in half of them), sparse rows, rows that start large or
    tiny (the sum's early binade crossings move), heavy-tailed values."""
    rng = np.random.default_rng(0xF022 + seed)
    x = np.zeros((rows, C), np.float32)
    for r in range(rows):
        v = rng.standard_normal(C) * 10.0 ** rng.uniform(-25, 25)
        if r % 2:
            v *= np.repeat(10.0 ** rng.uniform(-3, 3, C // 64), 64)
        if r % 5 == 0:
            v *= rng.random(C) < rng.uniform(0.001, 0.3)
        if r % 7 == 0:
            v[:rng.integers(1, 300)] *= 10.0 ** rng.uniform(-8, 8)
        if r % 11 == 0:
            v = rng.standard_cauchy(C)
        x[r] = v
    with np.errstate(over="ignore"):
        return bf16(x)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_rmsq_fuzz_rows_bit_exact(gpu, seed):
    """The parallel-sum kernel on fuzzed rows against the CPU oracle."""
    print(f"[case] rmsnorm_quant_256 fuzz seed={seed}", flush=True)
    x = fuzz_rows(seed=seed)
    g = I.uniform_bf16(I.SEED_BASE + 78 + seed, (C,), 0.25, 4.0)
    args = [x, g, np.zeros((256, C), np.int8), np.zeros(256, np.float32)]
    q, s = run_gpu("rmsnorm_quant_256", args, gpu)
    rq, rs = run_oracle("rmsnorm_quant_256", args)
    nan = np.isnan(rs)
    assert np.array_equal(np.isnan(s), nan)
    assert np.array_equal(s[~nan].view(np.uint32), rs[~nan].view(np.uint32)), \
        f"scales differ in rows {np.nonzero(s.view(np.uint32) != rs.view(np.uint32))[0][:16]}"
    bad = np.nonzero((q != rq).any(axis=1))[0]
    assert bad.size == 0, f"codes differ in rows {bad[:16]}"


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["rmsnorm_quant_256", "rmsnorm_quant_256_rowprog", "rmsnorm_quant_256_rmsn",
                                  "rmsnorm_quant_init"])
def test_rmsq_stress_rows_bit_exact(gpu, name):
    """The stress rows through the three kernels of the pattern: the
    parallel sum (hf_rmsq.h, the default), the generic row program and the
    opt-in chain-wave kernel (hf_rmsn.h, whose exact re-execution takes the
    NaN, infinite, overflowing and zero rows)."""
    print(f"[case] {name} stress rows", flush=True)
    x = stress_rows()
    g = I.uniform_bf16(I.SEED_BASE + 77, (C,), 0.5, 1.5)
    args = [x, g, np.zeros((256, C), np.int8), np.zeros(256, np.float32)]
    q, s = run_gpu(name, args, gpu)
    rq, rs = run_oracle("rmsnorm_quant_init" if name == "rmsnorm_quant_init" else "rmsnorm_quant_256", args)
    nan = np.isnan(rs)
    assert np.array_equal(np.isnan(s), nan)
    assert np.array_equal(s[~nan].view(np.uint32), rs[~nan].view(np.uint32)), \
        f"scales differ in rows {np.nonzero(s.view(np.uint32) != rs.view(np.uint32))[0][:16]}"
    bad = np.nonzero((q != rq).any(axis=1))[0]
    assert bad.size == 0, f"codes differ in rows {bad[:16]}"


def test_rmsq_kernel_selection():
    for name in ("rmsnorm_quant", "rmsnorm_quant_256", "rmsnorm_quant_rank3"):
        v = hf.compile(cat.get(name)).blocks[0]["variant"]
        assert "binade-run" in v, name
        v = hf.compile(cat.get(name), options="rmsq_kernel=1").blocks[0]["variant"]
        assert "binade-run" in v, name
        v = hf.compile(cat.get(name), options="rmsq_kernel=0").blocks[0]["variant"]
        assert v.startswith("row-resident, serial-order"), name
        v = hf.compile(cat.get(name), options="rmsn_kernel=1").blocks[0]["variant"]
        assert "serial-order" in v and "chain wave" in v, name
    assert "binade-run" in hf.compile(cat.get("rmsnorm_quant_init")).blocks[0]["variant"]
    assert "0x1.333334p-2f" in open(hf.compile(cat.get("rmsnorm_quant_init"), options="emit=hip").source).read()
    # widths the kernel does not take keep the generic row program
    for name in ("rmsnorm_quant_ragged", "rmsnorm_quant_w3072"):
        v = hf.compile(cat.get(name)).blocks[0]["variant"]
        assert "serial-order" in v, name
    assert "binade-run" in hf.compile(cat.get("rmsnorm_quant_w2048")).blocks[0]["variant"]


SHAPES = {"rmsnorm_quant_rowprog": (8192, 4096), "rmsnorm_quant_rank3_rowprog": (4, 64, 1024),
          "rmsnorm_quant_ragged_rmsq": (13, 1000), "rmsnorm_quant_rmsn": (8192, 4096),
          "rmsnorm_quant_rank3_rmsn": (4, 64, 1024), "rmsnorm_quant_rank3": (4, 64, 1024)}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(SHAPES))
def test_rmsq_configs_bit_exact(gpu, name):
    print(f"[case] {name}", flush=True)
    shape = SHAPES[name]
    rng = np.random.default_rng(11)
    x = bf16(rng.normal(0, 1, shape))
    g = bf16(rng.uniform(0.5, 1.5, shape[-1:]))
    args = [x, g, np.zeros(shape, np.int8), np.zeros(shape[:-1], np.float32)]
    q, s = run_gpu(name, args, gpu)
    rq, rs = run_oracle(name, args)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(q, rq)
