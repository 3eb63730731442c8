"""Shared helpers for the parity tests: run a catalog group on the GPU and
through the CPU oracle on the same inputs."""
import numpy as np

import hfusion_mi355x as hf
import group_catalog as cat
from oracle import interp


def np_of(elem):
    return interp.NP[elem]


def empty_like_param(p):
    return np.zeros(p["shape"], dtype=np_of(p["elem"]))


def to_dev(a, elem, device):
    import torch
    a = np.asarray(a)
    t = torch.from_numpy(a if a.flags.c_contiguous else a.copy(order="C"))  # rank 0 stays rank 0
    if elem in ("bf16", "f16"):
        t = t.view(torch.bfloat16 if elem == "bf16" else torch.float16)
    if elem in ("f8E4M3FN", "f8E5M2"):
        t = t.view(torch.uint8).view(torch.float8_e4m3fn if elem == "f8E4M3FN" else torch.float8_e5m2)
    if elem == "i8" and t.dtype == torch.uint8:
        t = t.view(torch.int8)  # ui8 in the IR: the same bytes
    return t.to(device)


def to_host(t, elem):
    import torch
    if elem in ("bf16", "f16"):
        t = t.view(torch.int16)
        return t.cpu().numpy().view(np.uint16)
    if elem in ("f8E4M3FN", "f8E5M2"):
        return t.view(torch.uint8).cpu().numpy()
    if elem == "i1":
        return t.cpu().numpy().astype(np.bool_)
    return t.cpu().numpy()


def run_gpu(name, inputs, device, func=None):
    """Runs prebuilt catalog group `name` on the GPU; `inputs` holds one numpy
    array per group argument (outputs' initial contents included)."""
    art = hf.compile(cat.get(name), options=cat.options(name), require_cached=True)
    grp = art.load(func)
    params = grp.meta["params"]
    devs = []
    for a, p in zip(inputs, params):
        devs.append(a if p["role"] == "scalar" else to_dev(a, p["elem"], device))
    out = grp(*devs)
    outs = out if isinstance(out, tuple) else (out,)
    import torch
    torch.cuda.synchronize()
    return [to_host(t, r["elem"]) for t, r in zip(outs, grp.meta["results"])]


def run_oracle(name, inputs, func=None, cast_semantics="declared"):
    return interp.run(cat.get(name), *inputs, func=func, cast_semantics=cast_semantics)


def bf16_ulp_diff(a, b):
    """|a - b| in bf16 units in the last place (same-sign finite values)."""
    ia = np.asarray(a, np.uint16).astype(np.int32)
    ib = np.asarray(b, np.uint16).astype(np.int32)
    # map sign-magnitude to a monotonic integer line
    ma = np.where(ia & 0x8000, -(ia & 0x7FFF), ia & 0x7FFF)
    mb = np.where(ib & 0x8000, -(ib & 0x7FFF), ib & 0x7FFF)
    return np.abs(ma - mb)


# --------------------------------------------- reference runner text format
# printData of bishengir/lib/ExecutionEngine/BiShengIRRunnerUtils.cpp:72-97:
# rank, sizes, then the elements; integers in decimal except int8, which is
# written as its raw byte; floats as "%.9e" of their float value.
def print_data(arr, elem):
    arr = np.asarray(arr)
    out = [str(arr.ndim)]
    if arr.ndim:
        out.append("\n" + " ".join(str(d) for d in arr.shape))
    flat = arr.reshape(-1)
    if elem == "bf16":
        vals = [f"{v:.9e}" for v in (flat.astype(np.uint32) << 16).view(np.float32)]
    elif elem in ("f32", "f64"):
        vals = [f"{v:.9e}" for v in flat.astype(np.float64 if elem == "f64" else np.float32)]
    elif elem == "f16":
        vals = [f"{v:.9e}" for v in flat.view(np.float16).astype(np.float32)]
    elif elem == "i8":
        vals = [bytes([int(v) & 0xFF]).decode("latin-1") for v in flat]
    elif elem == "i1":
        vals = [str(int(bool(v))) for v in flat]
    else:
        vals = [str(int(v)) for v in flat]
    body = "".join(("\n" if i == 0 else " ") + v for i, v in enumerate(vals))
    return ("".join(out) + body + "\n").encode("latin-1")


def parse_data_file(raw, elems, shapes):
    """Reads the tensors of a printData file back, given their element types
    and shapes (int8 elements are single raw bytes, so the layout is needed)."""
    pos, out = 0, []
    for elem, shape in zip(elems, shapes):
        n = int(np.prod(shape)) if shape else 1
        header = str(len(shape)) + ("\n" + " ".join(str(d) for d in shape) if shape else "")
        assert raw[pos:pos + len(header)].decode() == header, (raw[pos:pos + 40], header)
        pos += len(header)
        if elem == "i8":
            body = raw[pos:pos + 2 * n]
            vals = np.frombuffer(body[1::2], np.int8).copy()
            pos += 2 * n
        else:
            end = raw.index(b"\n", pos + 1)
            toks = raw[pos + 1:end].split(b" ")
            pos = end
            if elem in ("f32", "f64", "bf16", "f16"):
                f = np.array([float(t) for t in toks], np.float64)
                if elem == "bf16":
                    vals = (f.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
                elif elem == "f16":
                    vals = f.astype(np.float16).view(np.uint16)
                else:
                    vals = f.astype(np.float32 if elem == "f32" else np.float64)
            else:
                vals = np.array([int(t) for t in toks], np_of(elem))
        assert raw[pos:pos + 1] == b"\n"
        pos += 1
        out.append(vals.reshape(shape))
    assert pos == len(raw)
    return out


# ------------------------------------------------ inputs of the math_fns module
def _logu(rng, n, lo, hi):
    return np.exp(rng.uniform(np.log(lo), np.log(hi), n))


def math_inputs(func, n=4096, seed=0x4D415448):
    """Seeded operands for function `func` of catalog module math_fns, over
    the function's domain plus its edges (zeros, infinities, NaN, poles,
    out-of-domain points)."""
    rng = np.random.default_rng(seed + sum(map(ord, func)))
    sgn = lambda m: rng.choice([-1.0, 1.0], m)  # noqa: E731
    f32 = lambda a: np.asarray(a, np.float32)  # noqa: E731
    edges = [0.0, -0.0, np.inf, -np.inf, np.nan]
    if func.startswith("u_"):
        fn = func[2:]
        if fn == "tan":
            x = rng.uniform(-1.5, 1.5, n)
        elif fn in ("acos", "asin", "atanh"):
            x = rng.uniform(-1.0, 1.0, n)
            x[:6] = [1.0, -1.0, 1.0000001, -1.0000001, 0.5, -0.5]
        elif fn == "acosh":
            x = 1.0 + _logu(rng, n, 1e-6, 1e3)
            x[:3] = [1.0, 0.999, -2.0]
        elif fn in ("asinh", "atan", "sinh", "cosh", "tanh"):
            x = sgn(n) * _logu(rng, n, 1e-4, 100.0)
        elif fn == "lgamma":
            x = rng.uniform(-10.0, 30.0, n)
            x[:6] = [1.0, 2.0, -3.0, 0.5, 1e-3, 100.0]
        elif fn == "ilogb":
            x = sgn(n) * _logu(rng, n, 1e-44, 3e38)
        elif fn in ("sin", "cos"):
            x = rng.uniform(-1e3, 1e3, n)
        elif fn == "erf":
            x = rng.uniform(-5.0, 5.0, n)
        elif fn in ("log", "log2", "log10", "rsqrt"):
            x = _logu(rng, n, 1e-30, 1e30)
            x[:3] = [-1.0, 1.0, 4.0]
        elif fn == "log1p":
            x = np.concatenate([rng.uniform(-0.999, 1.0, n // 2), _logu(rng, n - n // 2, 1.0, 1e6)])
            x[:3] = [-1.0, -2.0, 1e-8]
        elif fn == "exp2":
            x = rng.uniform(-140.0, 130.0, n)
        elif fn == "expm1":
            x = rng.uniform(-20.0, 89.0, n)
            x[:2] = [1e-8, -1e-8]
        else:
            raise KeyError(func)
        x = f32(x)
        x[-len(edges):] = edges
        return [x, np.zeros(n, np.float32)]
    if func.startswith("b_"):
        fn = func[2:]
        if fn == "atan2":
            a, b = rng.normal(0, 10, n), rng.normal(0, 10, n)
            a[:4], b[:4] = [0.0, -0.0, 1.0, -1.0], [0.0, 0.0, 0.0, -0.0]
        elif fn == "ldexp":
            a = sgn(n) * _logu(rng, n, 1e-40, 1e38)
            b = np.floor(rng.uniform(-160, 160, n))
            b[:3] = [1e10, -1e10, np.nan]
        elif fn == "divfhp":
            a, b = rng.normal(0, 1e3, n), rng.normal(0, 1, n)
            b[:2] = [0.0, -0.0]
        elif fn == "powf":
            a, b = _logu(rng, n, 1e-3, 1e3), rng.uniform(-10.0, 10.0, n)
            a[:4], b[:4] = [-2.0, -2.0, 0.0, 1.0], [3.0, 0.5, -1.0, np.inf]
        elif fn == "copysign":
            a, b = rng.normal(0, 10, n), rng.normal(0, 1, n)
            b[:2] = [-0.0, 0.0]
        elif fn == "mod":
            a, b = rng.normal(0, 100, n), rng.normal(0, 10, n)
            b[:2] = [0.0, np.inf]
        else:
            raise KeyError(func)
        return [f32(a), f32(b), np.zeros(n, np.float32)]
    if func.startswith("i_"):
        fn, t = func[2:].rsplit("_", 1)
        dt = {"i8": np.int8, "i16": np.int16, "i32": np.int32}[t]
        info = np.iinfo(dt)
        if fn == "powi":
            a = rng.integers(-20, 21, n)
            b = rng.integers(-3, 16 if t == "i32" else 21, n)
            a[:4], b[:4] = [1, -1, -1, 0], [-5, -5, -4, 0]
        else:
            a = rng.integers(info.min, info.max + 1, n)
            b = rng.integers(info.min, info.max + 1, n)
            b[:4] = [0, 1, -1, 7]
        return [a.astype(dt), b.astype(dt), np.zeros(n, dt)]
    if func == "bitcast_add":
        a = rng.normal(0, 1e3, n).astype(np.float32).view(np.int32)
        b = rng.normal(0, 1e3, n).astype(np.float32).view(np.int32)
        return [a, b, np.zeros(n, np.float32)]
    raise KeyError(func)


def math_funcs():
    """Names of the functions of catalog module math_fns."""
    c = cat
    return ([f"u_{fn}" for fn, _ in c.MATH_UNARY] + [f"b_{fn}" for fn in c.MATH_BINARY]
            + [f"i_{fn}_{t}" for fn, t in c.INT_BINARY] + ["bitcast_add"])


# functions of math_fns whose result is exactly rounded (bit-exact bar)
MATH_EXACT = {"u_ilogb", "b_ldexp", "b_divfhp", "b_copysign", "b_mod", "bitcast_add"}


def fp_inputs(func, n=4096, seed=0x46504F50):
    """Seeded operands for group `func` of catalog module fp_ops, with
    specials (signed zeros, infinities, NaN, denormals, extremes)."""
    rng = np.random.default_rng(seed + sum(map(ord, func)))
    op, t = func.rsplit("_", 1)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 3.4e38, -3.4e38, 1.0], np.float32)

    def enc(f):
        f = np.asarray(f, np.float32)
        if t == "f32":
            return f
        if t == "f16":
            return f.astype(np.float16).view(np.uint16)
        if t == "bf16":
            return (f.view(np.uint32) >> 16).astype(np.uint16)  # truncation: exact bf16 values
        raise KeyError(t)
    if op == "cylbesseli0":
        x = rng.normal(0, 20, n).astype(np.float32)
        x[:len(specials)] = specials
        x[len(specials):len(specials) + 10] = [85.0, 92.0, -95.0, 100.5, 13.5, 1e-3, 89.0, -90.0, 91.0, 88.7228317]
        return [enc(x)]
    if op in ("isinf", "isnan", "isfinite", "signbit", "signbit8"):
        x = (rng.normal(0, 1e3, n)).astype(np.float32)
        x[:len(specials)] = specials
        x[rng.integers(0, n, 64)] = np.inf
        x[rng.integers(0, n, 64)] = np.nan
        x[rng.integers(0, n, 64)] = -np.nan
        return [enc(x)]
    if op == "nextafter":
        x = rng.normal(0, 10, n).astype(np.float32)
        y = rng.normal(0, 10, n).astype(np.float32)
        x[:len(specials)] = specials
        y[:len(specials)] = specials[::-1]
        x[20:30] = y[20:30]          # x == y
        x[30:34], y[30:34] = [0.0, -0.0, 0.0, 65504.0], [-1.0, 1.0, 0.0, np.inf]
        return [enc(x), enc(y)]
    if op in ("hypot", "hypot3"):
        k = 3 if op == "hypot3" else 2
        lim = 30 if t == "f32" else 4
        vs = [(rng.choice([-1.0, 1.0], n) * np.exp(rng.uniform(-lim, lim, n))).astype(np.float32) for _ in range(k)]
        vs[0][:6], vs[1][:6] = [0.0, np.inf, np.nan, 3.0, 1e-30, 1e30], [0.0, np.nan, 1.0, 4.0, 1e-30, 1e30]
        vs[0][6:10] = vs[1][6:10]    # equal magnitudes
        return [enc(v) for v in vs]
    if op == "erfinv":
        x = rng.uniform(-1.0, 1.0, n).astype(np.float32)
        x[:8] = [0.0, -0.0, 1.0, -1.0, 1.5, np.nan, 0.9999999, -1e-30]
        return [enc(x)]
    if op == "bitcast":
        return [rng.integers(-2**31, 2**31, n, dtype=np.int64).astype(np.int32), np.zeros(n, np.float32)]
    raise KeyError(func)


def fp_funcs():
    return [f"{op}_{t}" for op, t in cat.FP_OPS]


def scan_inputs(name, seed=0x5343414E):
    """Seeded input of group `name` of catalog module scan_ops."""
    spec = {s[0]: s for s in cat.SCAN_OPS}[name]
    _, op, ie, _, shape, _, _, _ = spec
    rng = np.random.default_rng(seed + sum(map(ord, name)))
    if ie in ("f32", "bf16"):
        if op == "cumprod":
            x = rng.uniform(0.9, 1.1, shape)
        else:
            x = rng.normal(0, 10, shape)
        x = x.astype(np.float32)
        flat = x.reshape(-1)
        if op in ("cummax", "cummin"):
            flat[rng.integers(0, flat.size, 40)] = np.nan
        if op == "cumprod":
            flat[rng.integers(0, flat.size, 8)] = 0.0
        if ie == "bf16":
            return [(x.view(np.uint32) >> 16).astype(np.uint16)]
        return [x]
    dt = {"i8": np.int8, "i16": np.int16, "i32": np.int32}[ie]
    lo, hi = {"cumprod": (-3, 4), "cumsum": (-2**31, 2**31), "cummax": (-128, 128)}[op]
    return [rng.integers(lo, hi, shape).astype(dt)]


def misc_inputs(name, seed=0x4D495343):
    """Seeded inputs of group `name` of catalog module misc_ops."""
    rng = np.random.default_rng(seed + sum(map(ord, name)))
    hist = {h[0]: h for h in cat.HIST_OPS}
    if name in hist:
        _, ie, shape, bins, _, me = hist[name]
        dt = {"i8": np.int8, "i32": np.int32}[ie]
        x = rng.integers(-5, bins + 5, shape).astype(dt)
        if me:
            return [x, rng.random(shape) < 0.7]
        return [x]
    _, e, ch = {i[0]: i for i in cat.INTERLEAVE_OPS}[name]
    def gen(shape):
        if e == "f32":
            return rng.normal(0, 1, shape).astype(np.float32)
        if e == "bf16":
            return rng.integers(0, 65536, shape).astype(np.uint16)
        return rng.integers(-128, 128, shape).astype(np.int8)
    if ch is None:
        return [gen((64, 500)), gen((64, 500))]
    return [gen((64, 1000))]


def misc_extra_inputs(name, seed=0x45585452):
    """Seeded arguments of the flip / mulext / arange groups of misc_ops."""
    rng = np.random.default_rng(seed + sum(map(ord, name)))
    if name.startswith("flip"):
        if name.endswith("bf16"):
            return [rng.integers(0, 65536, (64, 1000)).astype(np.uint16)]
        return [rng.normal(0, 1, (64, 1000)).astype(np.float32)]
    if name.startswith("mulext"):
        dt = {"i8": np.int8, "i32": np.int32, "i64": np.int64}[name.rsplit("_", 1)[1]]
        info = np.iinfo(dt)
        a = rng.integers(info.min, info.max, 4096, dtype=np.int64, endpoint=True).astype(dt)
        b = rng.integers(info.min, info.max, 4096, dtype=np.int64, endpoint=True).astype(dt)
        a[:4], b[:4] = [info.min, info.min, info.max, -1], [info.min, -1, info.max, -1]
        return [a, b]
    dt = np.int32 if name.endswith("i32") else np.float32
    return [np.zeros((48, 130), dt), np.int64(-77)]


def gather_inputs(name, seed=0x47415448):
    """Seeded (src, index, init) of group `name` of catalog module gather_ops;
    about one index in ten is out of range (negative or past the axis)."""
    spec = {g[0]: g for g in cat.GATHER_OPS}[name]
    _, se, ss, ie, ish, ax = spec
    rng = np.random.default_rng(seed + sum(map(ord, name)))
    src = rng.integers(0, 65536, ss).astype(np.uint16) if se in ("f16", "bf16") else rng.normal(0, 1, ss).astype(np.float32)
    if se == "f16":
        src = rng.normal(0, 1, ss).astype(np.float16).view(np.uint16)
    idx = rng.integers(-ss[ax] // 10, ss[ax] + ss[ax] // 10 + 1, ish).astype({"i32": np.int32, "i64": np.int64}[ie])
    init = np.full(ish, 0x7777 if se != "f32" else 7.0, src.dtype)
    return [src, idx, init]


def generic_inputs(name, seed=0x47454E45):
    """Seeded arguments of the groups of catalog module generic_ops."""
    rng = np.random.default_rng(seed + sum(map(ord, name)))
    if name == "generic_bias_act":
        return [rng.normal(0, 1, (64, 1000)).astype(np.float32), rng.normal(0, 1, 1000).astype(np.float32),
                rng.normal(0, 1, 64).astype(np.float32), np.float32(0.3), np.zeros((64, 1000), np.float32)]
    h = rng.normal(0, 2, (64, 1000)).astype(np.float16).view(np.uint16)
    i = rng.integers(-2**31, 2**31, (64, 1000), dtype=np.int64).astype(np.int32)
    i[:, :100] = rng.integers(-50, 50, (64, 100))
    return [h, i, np.zeros((64, 1000), np.uint16), np.zeros((64, 1000), np.bool_)]


def fuzz_inputs(n, seed=0x46555A5A):
    """Arguments of group fuzz<n> of catalog module fuzz_generic (its float
    type read from the group's signature)."""
    import re
    ir = cat.get("fuzz_generic")
    ft = re.search(r"@fuzz%d\(%%x: tensor<32x257x(\w+)>" % n, ir).group(1)
    rng = np.random.default_rng(seed + n)
    x = rng.normal(0, 3, (32, 257)).astype(np.float32)
    b = rng.normal(0, 3, 257).astype(np.float32)
    x[0, :4] = [0.0, -0.0, np.inf, np.nan]
    i = rng.integers(-100, 100, (32, 257)).astype(np.int32)
    if ft == "f16":
        x, b = x.astype(np.float16).view(np.uint16), b.astype(np.float16).view(np.uint16)
    return [x, b, i, np.zeros_like(x)], ft


def fuzz_row_inputs(n, seed=0x46524F57):
    """Arguments of group frow<n> of catalog module fuzz_rows (shape read
    from its signature), with ±0, ±inf and a NaN row among the values."""
    import re
    ir = cat.get("fuzz_rows")
    r, c = map(int, re.search(r"@frow%d\(%%x: tensor<(\d+)x(\d+)xf32>" % n, ir).groups())
    rng = np.random.default_rng(seed + n)
    x = rng.normal(0, 5, (r, c)).astype(np.float32)
    b = rng.normal(0, 5, c).astype(np.float32)
    x[0, :3] = [0.0, -0.0, np.inf]
    if r > 2:
        x[2, c // 2] = np.nan
    return [x, b, np.zeros(r, np.float32)]
