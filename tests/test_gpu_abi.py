"""GPU tests of the C-ABI entry points other than hfr_group_launch:

* hfr_group_launch_memref — MLIR ranked memref descriptors
  ({allocated, aligned, offset, sizes[R], strides[R]}, the `_mlir_ciface_*`
  argument layout) in the IR's argument order, with non-zero offsets;
* hfr_module_load -> hfr_kernel_get -> hfr_launch — the one-to-one
  replacements of rtDevBinaryRegister / rtFunctionRegister / rtKernelLaunch
  (bishengir/test/Integration/HIVM/VecAdd/main.cpp), driven by hand from a
  compiled group's code object and manifest.

Results are compared with the CPU oracle (bit-exact)."""
import ctypes
import os

import numpy as np
import pytest

import hfusion_mi355x as hf
import group_catalog as cat
from hfusion_mi355x import native
from helpers import run_oracle, to_dev, to_host

pytestmark = pytest.mark.gpu
I = hf.inputs


def note(msg):
    print(f"[case] {msg}", flush=True)


def _elem_size(elem):
    return {"f64": 8, "i64": 8, "f32": 4, "i32": 4, "f16": 2, "bf16": 2, "i16": 2}.get(elem, 1)


def _placed(a, elem, offset, device):
    """A device buffer holding `a` after `offset` elements of padding (filled
    with a marker byte), as (tensor, the buffer's base address)."""
    import torch
    t = to_dev(np.asarray(a), elem, device).reshape(-1).view(torch.uint8)
    pad = offset * _elem_size(elem)
    buf = torch.full((pad + t.numel() + 64,), 0xA5, dtype=torch.uint8, device=device)
    buf[pad:pad + t.numel()] = t
    return buf, buf.data_ptr()


def _read(buf, elem, shape, offset):
    import torch
    n = int(np.prod(shape)) if shape else 1
    pad = offset * _elem_size(elem)
    raw = buf[pad:pad + n * _elem_size(elem)]
    dt = {"f32": torch.float32, "i32": torch.int32, "i8": torch.int8, "i64": torch.int64,
          "bf16": torch.bfloat16, "f16": torch.float16}[elem]
    return to_host(raw.view(dt).reshape(shape), elem)


def test_memref_descriptors_with_offsets(gpu):
    """RMSNorm+quant group through hfr_group_launch_memref; every buffer sits
    at a different non-zero element offset behind its allocation."""
    note("memref rmsnorm_quant_ragged")
    import torch
    name, rows, cols = "rmsnorm_quant_ragged", 13, 1000
    x, gamma = I.config_inputs("rmsnorm_quant", rows=rows, cols=cols)
    args = [x, gamma, np.zeros((rows, cols), np.int8), np.zeros(rows, np.float32)]
    grp = hf.compile(cat.get(name), require_cached=True).load()
    params = grp.meta["params"]
    offs = [3, 7, 11, 5]
    bufs, descs = [], []
    for a, p, o in zip(args, params, offs):
        buf, base = _placed(a, p["elem"], o, gpu)
        bufs.append(buf)
        descs.append(native.memref_descriptor(base, list(p["shape"]), offset=o))
    ptrs = (ctypes.c_void_p * len(descs))(*[ctypes.addressof(d) for d in descs])
    torch.cuda.synchronize()
    native.check(native.hfr().hfr_group_launch_memref(grp._h, ptrs, len(descs), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    q = _read(bufs[2], "i8", (rows, cols), offs[2])
    s = _read(bufs[3], "f32", (rows,), offs[3])
    rq, rs = run_oracle(name, args)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(q, rq)
    # the padding in front of each output is untouched
    assert bool((bufs[2][:offs[2]] == 0xA5).all()) and bool((bufs[3][:4 * offs[3]] == 0xA5).all())


def test_memref_descriptor_untied_result_and_errors(gpu):
    """A result with its own buffer takes the descriptor after the arguments;
    wrong sizes, a written view that overlaps itself and a wrong descriptor
    count are refused."""
    note("memref reshape_chain")
    import torch
    s = I.SEED_BASE + 97
    args = [I.normal_f32(s, (128, 256)), I.normal_f32(s + 1, (128, 256)), I.normal_f32(s + 2, (32, 4, 256))]
    grp = hf.compile(cat.get("reshape_chain"), require_cached=True).load()
    assert [r["tied"] for r in grp.meta["results"]] == [-1]
    bufs, descs = [], []
    for k, (a, p) in enumerate(zip(args, grp.meta["params"])):
        buf, base = _placed(a, p["elem"], 2 + k, gpu)
        bufs.append(buf)
        descs.append(native.memref_descriptor(base, list(p["shape"]), offset=2 + k))
    res = grp.meta["results"][0]
    obuf, obase = _placed(np.zeros(res["shape"], np.float32), "f32", 9, gpu)
    descs.append(native.memref_descriptor(obase, list(res["shape"]), offset=9))
    ptrs = (ctypes.c_void_p * len(descs))(*[ctypes.addressof(d) for d in descs])
    stream = torch.cuda.current_stream().cuda_stream
    lib = native.hfr()
    torch.cuda.synchronize()
    native.check(lib.hfr_group_launch_memref(grp._h, ptrs, len(descs), stream))
    torch.cuda.synchronize()
    out = _read(obuf, "f32", res["shape"], 9)
    ref, = run_oracle("reshape_chain", args)
    assert np.array_equal(out, ref)
    # refusals (checked on the host, nothing is launched)
    assert lib.hfr_group_launch_memref(grp._h, ptrs, len(descs) - 1, stream) == -1
    bad = native.memref_descriptor(obase, [128, 255], offset=9)
    ptrs_bad = (ctypes.c_void_p * len(descs))(*([ctypes.addressof(d) for d in descs[:-1]] + [ctypes.addressof(bad)]))
    assert lib.hfr_group_launch_memref(grp._h, ptrs_bad, len(descs), stream) == -1
    assert b"size" in lib.hfr_last_error()
    # a written view that overlaps itself (stride 0 on a dim of 128)
    overl = native.memref_descriptor(obase, [128, 256], offset=9, strides=[0, 1])
    ptrs_st = (ctypes.c_void_p * len(descs))(*([ctypes.addressof(d) for d in descs[:-1]] + [ctypes.addressof(overl)]))
    assert lib.hfr_group_launch_memref(grp._h, ptrs_st, len(descs), stream) == -1
    assert b"overlaps" in lib.hfr_last_error()


def test_module_kernel_launch_by_hand(gpu):
    """hfr_module_load / hfr_kernel_get / hfr_launch on a compiled group's
    code object, with the launch shape and argument order of its manifest."""
    note("hfr_launch vec_add_ragged")
    import torch
    art = hf.compile(cat.get("vec_add_ragged"), require_cached=True)
    meta = art.blocks[0]
    hsaco = os.path.join(os.path.dirname(art.manifest), meta["hsaco"])
    lib = native.hfr()
    mod, ker = ctypes.c_void_p(), ctypes.c_void_p()
    native.check(lib.hfr_module_load(hsaco.encode(), ctypes.byref(mod)))
    try:
        native.check(lib.hfr_kernel_get(mod, meta["kernel"].encode(), ctypes.byref(ker)))
        assert lib.hfr_kernel_get(mod, b"no_such_kernel", ctypes.byref(ctypes.c_void_p())) == -5
        n = 1001
        a, b = I.config_inputs("vec_add", n=n)
        da, db = to_dev(a, "f32", gpu), to_dev(b, "f32", gpu)
        dout = torch.zeros(n, dtype=torch.float32, device=gpu)
        ptr = {"param:0": da.data_ptr(), "param:1": db.data_ptr(), "param:2": dout.data_ptr()}
        args = (ctypes.c_uint64 * len(meta["kargs"]))(*[ptr[k] for k in meta["kargs"]])
        cfg = native.LaunchCfg()
        for i in range(3):
            cfg.grid[i] = meta["grid"][i]
            cfg.block[i] = meta["block"][i]
        cfg.lds_bytes = meta.get("lds", 0)
        native.check(lib.hfr_launch(ker, ctypes.byref(cfg), args, len(meta["kargs"]),
                                    torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        ref, = run_oracle("vec_add_ragged", [a, b, np.zeros(n, np.float32)])
        assert np.array_equal(dout.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    finally:
        native.check(lib.hfr_module_unload(mod))


def _view_desc(view, base, dev_ptr):
    """Descriptor of numpy view `view` of `base`, addressed in the device copy
    of `base` at dev_ptr (element offset and strides as numpy has them)."""
    es = base.itemsize
    off = (view.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // es
    return native.memref_descriptor(dev_ptr, list(view.shape), offset=off, strides=[s // es for s in view.strides])


@pytest.mark.gpu
@pytest.mark.parametrize("x_transposed", [False, True])
def test_memref_strided_views(gpu, x_transposed):
    """Strided views at the GPU entry: x with a row pitch (or read through a
    transposed view), gamma with element stride 2, the int8 codes written
    through a transposed view and the scales at an offset.  The outputs equal
    the oracle's memref entry on the same descriptors over host copies, and
    no element outside the views is written."""
    note(f"memref strided rmsnorm_quant_ragged x_transposed={x_transposed}")
    import torch
    from oracle.interp import lib as oracle_lib, ptr as optr
    name, rows, cols = "rmsnorm_quant_ragged", 13, 1000
    x, gamma = I.config_inputs("rmsnorm_quant", rows=rows, cols=cols)
    if x_transposed:
        XB = np.zeros((cols + 7, rows + 3), np.uint16)
        XB[4:4 + cols, 1:1 + rows] = x.T
        xv = XB.T[1:1 + rows, 4:4 + cols]             # strides (1, rows + 3)
    else:
        XB = np.zeros((rows + 5, cols + 100), np.uint16)
        XB[2:2 + rows, 5:5 + cols] = x
        xv = XB[2:2 + rows, 5:5 + cols]               # row pitch 1100
    G = np.zeros(2 * cols + 3, np.uint16)
    G[1:1 + 2 * cols:2] = gamma
    gv = G[1:1 + 2 * cols:2]
    Q = np.full((cols + 10, rows + 7), 0x5A, np.int8)
    qv = Q.T[3:3 + rows, 6:6 + cols]                  # codes through a transposed view
    S = np.full(rows + 9, -1.0, np.float32)
    sv = S[4:4 + rows]
    assert np.array_equal(xv, x) and np.array_equal(gv, gamma)
    dXB, dG, dQ, dS = (torch.from_numpy(a.view(np.uint8).copy()).to(gpu) for a in (XB, G, Q, S))
    descs = [_view_desc(xv, XB, dXB.data_ptr()), _view_desc(gv, G, dG.data_ptr()),
             _view_desc(qv, Q, dQ.data_ptr()), _view_desc(sv, S, dS.data_ptr())]
    grp = hf.compile(cat.get(name), require_cached=True).load()
    ptrs = (ctypes.c_void_p * len(descs))(*[ctypes.addressof(d) for d in descs])
    torch.cuda.synchronize()
    native.check(native.hfr().hfr_group_launch_memref(grp._h, ptrs, len(descs), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    gQ = dQ.cpu().numpy().view(np.int8).reshape(Q.shape)
    gS = dS.cpu().numpy().view(np.float32)
    # the oracle's memref entry over host copies, same descriptors
    hQ, hS = Q.copy(), S.copy()
    L = oracle_lib()
    hdesc = [_view_desc(v, b, b.ctypes.data) for v, b in
             ((xv, XB), (gv, G), (hQ.T[3:3 + rows, 6:6 + cols], hQ), (hS[4:4 + rows], hS))]
    assert L.hfref_rmsnorm_quant_memref(*[ctypes.byref(d) for d in hdesc[:2]], ctypes.c_float(1e-6),
                                        *[ctypes.byref(d) for d in hdesc[2:]]) == 0
    assert np.array_equal(gQ, hQ), "codes (or the bytes around the view) differ"
    assert np.array_equal(gS.view(np.uint32), hS.view(np.uint32)), "scales (or the floats around the view) differ"
    rq, rs = run_oracle(name, [x, gamma, np.zeros((rows, cols), np.int8), np.zeros(rows, np.float32)])
    assert np.array_equal(gQ.T[3:3 + rows, 6:6 + cols], rq)
    outside = np.ones(Q.shape, bool)
    outside.T[3:3 + rows, 6:6 + cols] = False
    assert bool((gQ[outside] == 0x5A).all()) and bool((gS[:4] == -1.0).all()) and bool((gS[4 + rows:] == -1.0).all())


def test_group_launcher_repeats_the_launch(gpu):
    """Group.launcher: the arguments checked and packed once, then launched
    three times over new contents of the same buffers; each launch matches
    the oracle on the contents it saw (safe softmax rows, bf16 out, within
    the softmax bar of 1 bf16 ulp)."""
    import torch
    from helpers import bf16_ulp_diff
    note("launcher safe_softmax_ragged x3")
    art = hf.compile(cat.get("safe_softmax_ragged"), options=cat.options("safe_softmax_ragged"), require_cached=True)
    grp = art.load()
    p = grp.meta["params"]
    rows, cols = p[0]["shape"]
    x = to_dev(np.zeros((rows, cols), np.float32), p[0]["elem"], gpu)
    o = to_dev(np.zeros((rows, cols), np.uint16), p[1]["elem"], gpu)
    go = grp.launcher(x, o)
    for k in range(3):
        xs = I.normal_f32(I.SEED_BASE + 900 + k, (rows, cols), 2.0)
        x.copy_(torch.from_numpy(xs).to(gpu))
        go()
        torch.cuda.synchronize()
        ref, = run_oracle("safe_softmax_ragged", [xs, np.zeros((rows, cols), np.uint16)])
        d = bf16_ulp_diff(to_host(o, p[1]["elem"]), ref)
        assert d.max() <= 1, (k, int(d.max()))
