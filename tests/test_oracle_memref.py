"""The oracle's host-entry ABI: the group entries that take MLIR ranked memref
descriptors ({allocated, aligned, offset, sizes[R], strides[R]}, the
`_mlir_ciface_` argument layout of BiShengIRRunnerUtils.cpp:99-110), fed
views with offsets, element strides and transposes, agree with the dense
entries run on contiguous copies of the same views."""
import ctypes

import numpy as np
import pytest

from hfusion_mi355x.native import memref_descriptor
from oracle.interp import lib, ptr


def desc(view, base):
    """Descriptor of numpy view `view` of array `base` (element strides)."""
    es = base.itemsize
    off = (view.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // es
    st = [s // es for s in view.strides]
    assert all(s > 0 for s in st)
    return memref_descriptor(base.ctypes.data, view.shape, offset=off, strides=st)


def ref(d):
    return ctypes.byref(d)


def test_gather_scatter_roundtrip():
    L = lib()
    base = np.arange(7 * 11, dtype=np.int32).reshape(7, 11)
    v = base[1:6:2, 3:10:3]                          # offset 14, strides (22, 3)
    out = np.empty(v.shape, np.int32)
    assert L.hfref_memref_gather(ref(desc(v, base)), 2, 4, ptr(out)) == 0
    assert np.array_equal(out, v)
    b2 = np.zeros_like(base)
    assert L.hfref_memref_scatter(ptr(out * 2), ref(desc(b2[1:6:2, 3:10:3], b2)), 2, 4) == 0
    assert np.array_equal(b2[1:6:2, 3:10:3], v * 2) and b2.sum() == (v * 2).sum()


def test_vecadd_memref_strided():
    L = lib()
    rng = np.random.default_rng(1)
    A = rng.standard_normal(300).astype(np.float32)
    B = rng.standard_normal(600).astype(np.float32)
    O = np.zeros(400, np.float32)
    a, b, o = A[7:107], B[1:201:2], O[50:150]
    assert L.hfref_vecadd_f32_memref(ref(desc(a, A)), ref(desc(b, B)), ref(desc(o, O))) == 0
    want = np.empty(100, np.float32)
    L.hfref_vecadd_f32(ptr(np.ascontiguousarray(a)), ptr(np.ascontiguousarray(b)), ptr(want), 100)
    assert np.array_equal(o.view(np.uint32), want.view(np.uint32))
    assert not O[:50].any() and not O[150:].any()


def test_rmsnorm_quant_memref_views():
    L = lib()
    rng = np.random.default_rng(2)
    X = rng.standard_normal((40, 300)).astype(np.float32)
    Xb = (X.view(np.uint32) >> 16).astype(np.uint16)
    G = (rng.uniform(0.5, 1.5, 600).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    Q = np.zeros((300, 40), np.int8)                 # q written through a transposed view
    S = np.zeros(100, np.float32)
    x, g, q, s = Xb[3:35, 10:266], G[0:512:2], Q.T[3:35, 10:266], S[5:37]
    assert L.hfref_rmsnorm_quant_memref(ref(desc(x, Xb)), ref(desc(g, G)), ctypes.c_float(1e-6),
                                        ref(desc(q, Q)), ref(desc(s, S))) == 0
    wq, ws = np.empty((32, 256), np.int8), np.empty(32, np.float32)
    L.hfref_rmsnorm_quant(ptr(np.ascontiguousarray(x)), ptr(np.ascontiguousarray(g)), ctypes.c_float(1e-6),
                          ptr(wq), ptr(ws), 32, 256)
    assert np.array_equal(q, wq) and np.array_equal(s.view(np.uint32), ws.view(np.uint32))


def test_softmax_argmax_w8a8_memref():
    L = lib()
    rng = np.random.default_rng(3)
    X = rng.standard_normal((64, 48)).astype(np.float32)
    x = X.T[4:36]                                    # [32, 64] transposed view
    O = np.zeros((32, 80), np.uint16)
    assert L.hfref_softmax_bf16_memref(ref(desc(x, X)), ref(desc(O[:, 8:72], O))) == 0
    w = np.empty((32, 64), np.uint16)
    L.hfref_softmax_bf16(ptr(np.ascontiguousarray(x)), ptr(w), 32, 64)
    assert np.array_equal(O[:, 8:72], w)

    V, I = np.zeros(40, np.float32), np.zeros(40, np.int32)
    assert L.hfref_argmax_memref(ref(desc(x, X)), ref(desc(V[2:34], V)), ref(desc(I[4:36], I))) == 0
    wv, wi = np.empty(32, np.float32), np.empty(32, np.int32)
    L.hfref_argmax(ptr(np.ascontiguousarray(x)), ptr(wv), ptr(wi), 32, 64)
    assert np.array_equal(V[2:34], wv) and np.array_equal(I[4:36], wi)

    # B stored [K, N] and passed as its [N, K] transposed view: the weight
    # layout through strides alone
    M, N, K = 24, 40, 96
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    BKN = rng.integers(-128, 128, (K, N), dtype=np.int8)
    st = rng.uniform(0.001, 0.02, M).astype(np.float32)
    sc = rng.uniform(0.001, 0.02, N).astype(np.float32)
    OUT = np.zeros((M, N), np.uint16)
    assert L.hfref_w8a8_dequant_memref(ref(desc(A, A)), ref(desc(BKN.T, BKN)), ref(desc(st, st)),
                                       ref(desc(sc, sc)), ref(desc(OUT, OUT))) == 0
    wo = np.empty((M, N), np.uint16)
    L.hfref_w8a8_dequant_rows(ptr(A), ptr(np.ascontiguousarray(BKN.T)), ptr(st), ptr(sc), ptr(wo), M, N, K, 0, M)
    assert np.array_equal(OUT, wo)


def test_memref_shape_mismatch_is_an_error():
    L = lib()
    a = np.zeros(10, np.float32)
    b = np.zeros(11, np.float32)
    assert L.hfref_vecadd_f32_memref(ref(desc(a, a)), ref(desc(b, b)), ref(desc(a, a))) == -1
