"""GPU parity at BASELINE.json's full sizes.

Each configured group runs through the C-ABI runtime on its full synthetic
input.  Where the oracle's composed C loops finish in seconds, the whole
output is compared with them, to the bar of tests/test_gpu_parity.py.  For
the 4096^3 contraction (7e10 multiply-adds, minutes in the oracle) the checks
are size-independent instead: exact integer row and column checksums of the
raw int32 accumulator over the whole matrix, the full comparison of 64 spread
rows (every 256x256 tile row and column), and for the dequantised group the
same 64 rows bit-exact against the oracle.
"""
import numpy as np
import pytest

import hfusion_mi355x as hf
from helpers import bf16_ulp_diff, run_gpu
from oracle.interp import lib, ptr

pytestmark = pytest.mark.gpu
I = hf.inputs
CFG = hf.groups.CONFIGS


def note(msg):
    print(f"[case] {msg}", flush=True)


def test_vec_add_full(gpu):
    note("vec_add full [2^24]")
    a, b = I.config_inputs("vec_add", **CFG["vec_add"]["kw"])
    out, = run_gpu("vec_add", [a, b, np.zeros_like(a)], gpu)
    ref = np.empty_like(a)
    lib().hfref_vecadd_f32(ptr(a), ptr(b), ptr(ref), a.size)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_rmsnorm_quant_full(gpu):
    note("rmsnorm_quant full [8192, 4096]")
    kw = CFG["rmsnorm_quant"]["kw"]
    x, g = I.config_inputs("rmsnorm_quant", **kw)
    r, c = x.shape
    q, s = run_gpu("rmsnorm_quant", [x, g, np.zeros((r, c), np.int8), np.zeros(r, np.float32)], gpu)
    rq, rs = np.empty((r, c), np.int8), np.empty(r, np.float32)
    import ctypes
    lib().hfref_rmsnorm_quant(ptr(x), ptr(g), ctypes.c_float(kw["eps"]), ptr(rq), ptr(rs), r, c)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32)), "per-row scales must be bit-exact"
    assert np.array_equal(q, rq), f"{int((q != rq).sum())} int8 codes differ"


def test_safe_softmax_full(gpu):
    note("safe_softmax full [4096, 32768]")
    x, = I.config_inputs("safe_softmax", **CFG["safe_softmax"]["kw"])
    out, = run_gpu("safe_softmax", [x, np.zeros(x.shape, np.uint16)], gpu)
    ref = np.empty(x.shape, np.uint16)
    lib().hfref_softmax_bf16(ptr(x), ptr(ref), x.shape[0], x.shape[1])
    d = bf16_ulp_diff(out, ref)
    assert d.max() <= 1, f"max {d.max()} bf16 ulp"


def test_argmax_full(gpu):
    note("argmax full [256, 152064]")
    x, = I.config_inputs("argmax", **CFG["argmax"]["kw"])
    r = x.shape[0]
    v, i = run_gpu("argmax", [x, np.zeros(r, np.float32), np.zeros(r, np.int32)], gpu)
    rv, ri = np.empty(r, np.float32), np.empty(r, np.int32)
    lib().hfref_argmax(ptr(x), ptr(rv), ptr(ri), r, x.shape[1])
    assert np.array_equal(i, ri)
    assert np.array_equal(v.view(np.uint32), rv.view(np.uint32))


SAMPLE_ROWS = np.arange(64) * 64 + (np.arange(64) * 37) % 64  # one row in every 64, varying offset


def test_mm_i8_full_checksums(gpu):
    note("mm_i8 full 4096^3 int32 accumulator")
    kw = CFG["w8a8_dequant"]["kw"]
    a, b, _, _ = I.config_inputs("w8a8_dequant", **kw)
    m, n = a.shape[0], b.shape[0]
    c, = run_gpu("mm_i8_full", [a, b, np.zeros((m, n), np.int32)], gpu)
    a64, b64 = a.astype(np.int64), b.astype(np.int64)
    # row sums C 1 = A (B^T 1) and column sums 1^T C = (1^T A) B^T, exact in int64
    assert np.array_equal(c.astype(np.int64).sum(axis=1), a64 @ b64.sum(axis=0))
    assert np.array_equal(c.astype(np.int64).sum(axis=0), b64 @ a64.sum(axis=0))
    # 64 spread rows in full (float64 products and sums are exact: |C| < 2^53)
    rows = SAMPLE_ROWS
    assert np.array_equal(c[rows].astype(np.float64), a[rows].astype(np.float64) @ b.astype(np.float64).T)


def test_w8a8_dequant_full_sampled(gpu):
    note("w8a8_dequant full 4096^3, 64 sampled rows")
    kw = CFG["w8a8_dequant"]["kw"]
    a, b, st, sc = I.config_inputs("w8a8_dequant", **kw)
    m, n, k = a.shape[0], b.shape[0], a.shape[1]
    out, = run_gpu("w8a8_dequant", [a, b, st, sc, np.zeros((m, n), np.uint16)], gpu)
    ref = np.zeros((m, n), np.uint16)
    for r in SAMPLE_ROWS:
        lib().hfref_w8a8_dequant_rows(ptr(a), ptr(b), ptr(st), ptr(sc), ptr(ref), m, n, k, int(r), int(r) + 1)
    assert np.array_equal(out[SAMPLE_ROWS], ref[SAMPLE_ROWS])


def test_w8a8_dequant_kn_full_sampled(gpu):
    """W8A8 with B stored [K, N] (linalg.matmul): the DMA ring stages whole
    k-rows of B and forms the matrix-core operand with transposing LDS reads;
    64 sampled rows bit-exact against the oracle fed B^T."""
    note("w8a8_dequant_kn full 4096^3 (B [K,N]), 64 sampled rows")
    kw = CFG["w8a8_dequant"]["kw"]
    a, b, st, sc = I.config_inputs("w8a8_dequant", **kw)
    m, n, k = a.shape[0], b.shape[0], a.shape[1]
    bkn = np.ascontiguousarray(b.T)
    out, = run_gpu("w8a8_dequant_kn", [a, bkn, st, sc, np.zeros((m, n), np.uint16)], gpu)
    ref = np.zeros((m, n), np.uint16)
    for r in SAMPLE_ROWS:
        lib().hfref_w8a8_dequant_rows(ptr(a), ptr(b), ptr(st), ptr(sc), ptr(ref), m, n, k, int(r), int(r) + 1)
    assert np.array_equal(out[SAMPLE_ROWS], ref[SAMPLE_ROWS])
