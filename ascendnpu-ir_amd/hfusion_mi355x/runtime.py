"""Host-side mirror of the reference's compile-then-launch flow for HFusion groups.

Reference flow: ``bishengir-compile in.mlir -o kernel.o`` (device compile,
``bishengir/tools/bishengir-compile/bishengir-compile.cpp:103-191``), then the
host registers the binary and launches it with bare device pointers in the
kernel's argument order (``bishengir/test/Integration/HIVM/VecAdd/main.cpp``).
Here: ``compile(ir)`` runs the same lowering through libhfc (hipcc for gfx950)
and ``Group.__call__`` launches through libhfr on the current HIP stream.
PyTorch only supplies device memory and the stream.
"""
import ctypes
import hashlib
import os
import struct

from . import native

_DTYPES = None


def torch_dtype(elem):
    global _DTYPES
    import torch
    if _DTYPES is None:
        _DTYPES = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f64": torch.float64,
                   "i1": torch.bool, "i8": torch.int8, "i16": torch.int16, "i32": torch.int32,
                   "i64": torch.int64, "index": torch.int64, "f8E4M3FN": torch.float8_e4m3fn,
                   "f8E5M2": torch.float8_e5m2}
    return _DTYPES[elem]


CACHE_DIR = os.path.join(native.PKG_ROOT, "build", "kcache")


class CompileError(RuntimeError):
    pass


def _key(ir_text, options):
    h = hashlib.sha1()
    h.update(ir_text.encode())
    h.update(b"\0" + options.encode())
    # the kernel library and compiler sources are part of the key
    for d in (native.KERNEL_INCLUDE, os.path.join(native.PKG_ROOT, "csrc", "compiler")):
        for fn in sorted(os.listdir(d)):
            with open(os.path.join(d, fn), "rb") as f:
                h.update(fn.encode() + f.read())
    return h.hexdigest()[:20]


class Artifact:
    """Compiled group(s) of one IR module: P.hip / P.hsaco / P.manifest."""

    def __init__(self, prefix):
        self.prefix = prefix
        self.manifest = prefix + ".manifest"
        self.hsaco = prefix + ".hsaco"
        self.source = prefix + ".hip"
        self.blocks, self.programs = parse_manifest(self.manifest, with_programs=True)
        outlined = prefix + ".outlined.mlir"
        self.outlined = outlined if os.path.exists(outlined) else None

    def funcs(self):
        return [b["func"] for b in self.blocks]

    def program_names(self):
        return [p["name"] for p in self.programs]

    def load(self, func=None):
        """The group kernel named `func`, or, when `func` names a function the
        fusion front-end split (or is None and the module was split into
        exactly one program), its launch program."""
        if self.programs and (func is None or func in self.program_names()):
            return Program(self, func)
        return Group(self, func)


def compile(ir_text, options="", cache=True, require_cached=False):
    """Compiles IR text (one or more `hacc.entry` groups) to a gfx950 code object."""
    prefix = os.path.join(CACHE_DIR, _key(ir_text, options), "group")
    if cache and os.path.exists(prefix + ".hsaco") and os.path.exists(prefix + ".manifest"):
        return Artifact(prefix)
    if require_cached:
        raise CompileError(f"group not prebuilt (expected {prefix}.hsaco); run __graft_entry__.build()")
    os.makedirs(os.path.dirname(prefix), exist_ok=True)
    err = ctypes.create_string_buffer(16384)
    opts = f"include={native.KERNEL_INCLUDE};" + options
    rc = native.hfc().hfc_compile(ir_text.encode(), prefix.encode(), opts.encode(), err, len(err))
    if rc != 0:
        raise CompileError(err.value.decode(errors="replace"))
    return Artifact(prefix)


def _shape(parts, at):
    n = int(parts[at])
    return tuple(int(x) for x in parts[at + 1:at + 1 + n])


def parse_manifest(path, with_programs=False):
    blocks, programs = [], []
    cur = None
    with open(path) as f:
        for ln in f:
            ln = ln.rstrip("\n")
            if not ln:
                continue
            if ln.startswith("hfr-manifest"):
                cur = {"params": [], "results": [], "kargs": []}
                blocks.append(cur)
                continue
            if ln.startswith("hfr-program"):
                cur = {"params": [], "results": [], "temps": [], "steps": [], "program": True}
                programs.append(cur)
                continue
            key, _, rest = ln.partition(" ")
            b = cur
            parts = rest.split()
            if b.get("program"):
                if key == "program":
                    b["name"] = rest
                elif key == "pworkspace":
                    b["workspace"] = int(parts[0])
                elif key == "pparam":
                    b["params"].append(dict(role=parts[1], elem=parts[2], shape=_shape(parts, 3)))
                elif key == "presult":
                    role = parts[1]
                    b["results"].append(dict(tied=int(role[1:]) if role.startswith("p") else -1, elem=parts[2],
                                             shape=_shape(parts, 3)))
                elif key == "ptemp":
                    b["temps"].append(dict(offset=int(parts[1]), bytes=int(parts[2]), elem=parts[3],
                                           shape=_shape(parts, 4)))
                elif key == "pstep":
                    na = int(parts[2])
                    args = parts[3:3 + na]
                    nr = int(parts[3 + na])
                    b["steps"].append(dict(group=parts[0], kind=parts[1], args=args,
                                           results=parts[4 + na:4 + na + nr]))
                continue
            if key in ("func", "kernel", "hsaco", "kind"):
                b[key] = rest
            elif key == "variant":
                b[key] = rest
            elif key in ("grid", "block"):
                b[key] = tuple(int(x) for x in parts)
            elif key in ("lds", "algo_bytes", "algo_ops"):
                b[key] = int(parts[0])
            elif key == "workspace":
                b["workspace"] = int(parts[0])
                b["workspace_zero"] = bool(int(parts[1]))
            elif key == "param":
                b["params"].append(dict(role=parts[1], elem=parts[2], shape=_shape(parts, 3)))
            elif key == "result":
                b["results"].append(dict(tied=int(parts[1]), elem=parts[2], shape=_shape(parts, 3)))
            elif key == "karg":
                b["kargs"].append(parts[0])
            elif key == "rows_dyn":
                b["rows_dyn"] = tuple(int(x) for x in parts)
            elif key == "pre":
                b.setdefault("pre", []).append(dict(kernel=parts[0], grid=tuple(int(x) for x in parts[1:4]),
                                                    block=tuple(int(x) for x in parts[4:7]), kargs=parts[8:]))
    return (blocks, programs) if with_programs else blocks


def _scalar_bits(v, elem):
    if elem == "f32":
        return struct.unpack("<I", struct.pack("<f", float(v)))[0]
    if elem == "f64":
        return struct.unpack("<Q", struct.pack("<d", float(v)))[0]
    return int(v) & 0xFFFFFFFFFFFFFFFF


class Group:
    """One loaded HFusion group kernel (hfr_group_t)."""

    def __init__(self, artifact, func=None):
        blocks = artifact.blocks
        if func is None:
            if len(blocks) != 1:
                raise ValueError("artifact holds several groups; name one of " + ", ".join(artifact.funcs()))
            self.meta = blocks[0]
        else:
            match = [b for b in blocks if b["func"] == func]
            if not match:
                raise ValueError(f"no group @{func} in {artifact.manifest}")
            self.meta = match[0]
        self.func = self.meta["func"]
        self._h = ctypes.c_void_p()
        native.check(native.hfr().hfr_group_load(artifact.manifest.encode(), self.func.encode(), ctypes.byref(self._h)))
        info = native.GroupInfo()
        native.check(native.hfr().hfr_group_info_get(self._h, ctypes.byref(info)))
        self.info = info

    @property
    def algo_bytes(self):
        return self.meta.get("algo_bytes", 0)

    @property
    def algo_ops(self):
        return self.meta.get("algo_ops", 0)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and h.value and native._hfr is not None:
            native.hfr().hfr_group_unload(h)
            self._h = None

    def __call__(self, *args, results=None, stream=None, workspace=None, noalloc=False):
        """Launches the group on `stream` (torch's current stream by default).
        noalloc=True goes through hfr_group_launch_noalloc (the library's
        static scratch instead of a workspace)."""
        return self._bind(args, results, stream, workspace, noalloc)()

    def launcher(self, *args, results=None, stream=None, workspace=None, noalloc=False):
        """The launch of __call__ with its arguments checked and packed once:
        returns a callable that only enqueues the kernels (for loops that
        launch the same buffers many times)."""
        fn = self._bind(args, results, stream, workspace, noalloc)
        return lambda: fn()

    def _bind(self, args, results, stream, workspace, noalloc):
        import torch
        params = self.meta["params"]
        if len(args) != len(params):
            raise TypeError(f"@{self.func} takes {len(params)} arguments ({len(args)} given)")
        # a runtime row count (-1 row dims in the manifest): read from the
        # arguments, which must agree
        dyn = "rows_dyn" in self.meta
        rows = None
        for i, (a, p) in enumerate(zip(args, params)):
            if dyn and p["role"] != "scalar" and -1 in p["shape"] and isinstance(a, torch.Tensor):
                r = int(a.shape[p["shape"].index(-1)]) if a.dim() == len(p["shape"]) else -1
                if rows is not None and r != rows:
                    raise ValueError(f"argument {i} of @{self.func} has {r} rows, an earlier one {rows}")
                rows = r
        if dyn and rows is None:
            raise ValueError(f"@{self.func} takes its row count from a tensor argument")

        def want(shape):
            return tuple(rows if d == -1 else d for d in shape)
        device = None
        slots = (ctypes.c_uint64 * len(params))()
        for i, (a, p) in enumerate(zip(args, params)):
            if p["role"] == "scalar":
                slots[i] = _scalar_bits(a, p["elem"])
                continue
            if not isinstance(a, torch.Tensor) or not a.is_cuda:
                raise TypeError(f"argument {i} of @{self.func} must be a device tensor")
            if a.dtype != torch_dtype(p["elem"]) or tuple(a.shape) != want(p["shape"]) or not a.is_contiguous():
                raise ValueError(f"argument {i} of @{self.func}: expected contiguous "
                                 f"{p['elem']}{list(want(p['shape']))}, got {a.dtype}{list(a.shape)}")
            device = a.device if device is None else device
            slots[i] = a.data_ptr()
        res_meta = self.meta["results"]
        outs = []
        rptrs = (ctypes.c_void_p * max(1, len(res_meta)))()
        for j, r in enumerate(res_meta):
            if r["tied"] >= 0:
                outs.append(args[r["tied"]])
                rptrs[j] = None
            else:
                t = results[j] if results is not None else torch.empty(want(r["shape"]), dtype=torch_dtype(r["elem"]),
                                                                      device=device)
                if tuple(t.shape) != want(r["shape"]) or t.dtype != torch_dtype(r["elem"]) or not t.is_cuda:
                    raise ValueError(f"result {j} of @{self.func}: expected {r['elem']}{list(want(r['shape']))}")
                outs.append(t)
                rptrs[j] = t.data_ptr()
        if stream is None:
            stream = torch.cuda.current_stream(device).cuda_stream
        ret = outs[0] if len(outs) == 1 else tuple(outs)
        lib, h, n, nr = native.hfr(), self._h, len(params), len(res_meta)
        if noalloc:
            if workspace is not None:
                raise ValueError("noalloc launches take no workspace")

            def launch():
                native.check(lib.hfr_group_launch_noalloc(h, slots, n, rptrs, nr, stream))
                return ret
        elif dyn:
            ws = workspace.data_ptr() if workspace is not None else None

            def launch():
                native.check(lib.hfr_group_launch_rows(h, slots, n, rptrs, nr, rows, ws, stream))
                return ret
        else:
            ws = workspace.data_ptr() if workspace is not None else None

            def launch():
                native.check(lib.hfr_group_launch(h, slots, n, rptrs, nr, ws, stream))
                return ret
        return launch


def _check_arg(i, a, p, name):
    import torch
    if not isinstance(a, torch.Tensor) or not a.is_cuda:
        raise TypeError(f"argument {i} of @{name} must be a device tensor")
    if a.dtype != torch_dtype(p["elem"]) or tuple(a.shape) != p["shape"] or not a.is_contiguous():
        raise ValueError(f"argument {i} of @{name}: expected contiguous {p['elem']}{list(p['shape'])}, "
                         f"got {a.dtype}{list(a.shape)}")


class Program:
    """A function the fusion front-end split into fused groups (hfr_program_t):
    one call launches every group kernel in order on the current stream."""

    def __init__(self, artifact, name=None):
        progs = artifact.programs
        if name is None:
            if len(progs) != 1:
                raise ValueError("artifact holds several programs; name one of " + ", ".join(artifact.program_names()))
            self.meta = progs[0]
        else:
            self.meta = [p for p in progs if p["name"] == name][0]
        self.name = self.meta["name"]
        self.steps = self.meta["steps"]
        self._h = ctypes.c_void_p()
        native.check(native.hfr().hfr_program_load(artifact.manifest.encode(), self.name.encode(),
                                                   ctypes.byref(self._h)))
        info = native.ProgramInfo()
        native.check(native.hfr().hfr_program_info_get(self._h, ctypes.byref(info)))
        self.info = info

    @property
    def workspace_bytes(self):
        return self.info.workspace_bytes

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and h.value and native._hfr is not None:
            native.hfr().hfr_program_unload(h)
            self._h = None

    def __call__(self, *args, results=None, stream=None, workspace=None):
        """Launches the program's groups in order on `stream` (torch's current
        stream by default) through hfr_program_launch; intermediate tensors
        live in `workspace` (the program's own when None).  Programs have no
        no-allocation entry."""
        import torch
        params = self.meta["params"]
        if len(args) != len(params):
            raise TypeError(f"@{self.name} takes {len(params)} arguments ({len(args)} given)")
        device = None
        slots = (ctypes.c_uint64 * max(1, len(params)))()
        for i, (a, p) in enumerate(zip(args, params)):
            if p["role"] == "scalar":
                slots[i] = _scalar_bits(a, p["elem"])
                continue
            _check_arg(i, a, p, self.name)
            device = a.device if device is None else device
            slots[i] = a.data_ptr()
        res_meta = self.meta["results"]
        outs = []
        rptrs = (ctypes.c_void_p * max(1, len(res_meta)))()
        for j, r in enumerate(res_meta):
            if r["tied"] >= 0:
                outs.append(args[r["tied"]])
                rptrs[j] = None
            else:
                t = results[j] if results is not None else torch.empty(r["shape"], dtype=torch_dtype(r["elem"]),
                                                                      device=device)
                if tuple(t.shape) != r["shape"] or t.dtype != torch_dtype(r["elem"]) or not t.is_cuda:
                    raise ValueError(f"result {j} of @{self.name}: expected {r['elem']}{list(r['shape'])}")
                outs.append(t)
                rptrs[j] = t.data_ptr()
        if stream is None:
            stream = torch.cuda.current_stream(device).cuda_stream
        if workspace is not None and workspace.numel() * workspace.element_size() < self.workspace_bytes:
            raise ValueError(f"@{self.name} needs a workspace of {self.workspace_bytes} bytes")
        ws = workspace.data_ptr() if workspace is not None else None
        native.check(native.hfr().hfr_program_launch(self._h, slots, len(params), rptrs, len(res_meta), ws, stream))
        return outs[0] if len(outs) == 1 else tuple(outs)


def load(ir_text, func=None, options="", require_cached=False):
    """compile() + load(): the one-call host entry."""
    return compile(ir_text, options=options, require_cached=require_cached).load(func)


def _split_args(sig):
    """Top-level comma split of a func signature's argument list."""
    out, depth, cur = [], 0, ""
    for c in sig:
        if c in "<({[":
            depth += 1
        elif c in ">)}]":
            depth -= 1
        if c == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += c
    if cur.strip():
        out.append(cur)
    return out


def dynamic_dims(ir_text, func=None):
    """[(func, arg, dim)] of every dynamic (`?`) dim of the arguments of the
    module's functions (of `func` only when given), in argument order."""
    import re
    dims = []
    for m in re.finditer(r"func\.func\s+(?:private\s+)?@([\w.$-]+)\s*\(", ir_text):
        name = m.group(1)
        if func is not None and name != func:
            continue
        depth, i = 1, m.end()
        while depth:
            depth += {"(": 1, ")": -1}.get(ir_text[i], 0)
            i += 1
        for a, arg in enumerate(_split_args(ir_text[m.end():i - 1])):
            t = re.search(r"(?:tensor|memref)<([^>]*)>", arg)
            if not t:
                continue
            shape = t.group(1).split(",")[0].replace(" ", "").split("x")[:-1]
            dims += [(name, a, d) for d, s in enumerate(shape) if s == "?"]
    return dims


class DynamicGroup:
    """A group whose IR has dynamic (`?`) dims.

    Per size set (the default): the sizes of the dynamic argument dims are
    read from the tensors of each call; the group is specialised to them
    (compiler option `dyn=<func>:<arg>.<dim>=<size>,...`: every type of the
    function becomes static) and compiled once per size set, content-cached
    like any group.  A serving loop that buckets its sizes compiles each
    bucket once.  With `require_cached`, a size set that was not prebuilt
    raises instead of compiling.

    runtime=True: one kernel for every row count (compiler option
    `dyn=runtime`), for groups whose dynamic dims are all the row count
    (dim 0 of the arguments) and whose kernel takes it at launch (row
    programs, the RMSNorm + quant kernel, streaming elementwise groups of
    rank 2 and more, contractions whose M is the row count, reduce_with_index
    over rows); the compiler refuses the others."""

    def __init__(self, ir_text, func=None, options="", require_cached=False, runtime=False):
        self.ir_text, self.func, self.options, self.require_cached = ir_text, func, options, require_cached
        self.dims = dynamic_dims(ir_text, func)
        if not self.dims:
            raise ValueError("the group has no dynamic dims; use load()")
        self._groups = {}
        self._rt = None
        if runtime:
            opts = (options + ";" if options else "") + "dyn=runtime"
            self._rt = compile(ir_text, options=opts, require_cached=require_cached).load(func)

    def options_for(self, sizes):
        spec = ",".join(f"{f}:{a}.{d}={int(s)}" for (f, a, d), s in zip(self.dims, sizes))
        return (self.options + ";" if self.options else "") + "dyn=" + spec

    def sizes_of(self, args):
        return tuple(int(args[a].shape[d]) for _, a, d in self.dims)

    def specialise(self, sizes):
        if self._rt is not None:
            return self._rt
        sizes = tuple(int(s) for s in sizes)
        if sizes not in self._groups:
            art = compile(self.ir_text, options=self.options_for(sizes), require_cached=self.require_cached)
            self._groups[sizes] = art.load(self.func)
        return self._groups[sizes]

    def __call__(self, *args, **kw):
        if self._rt is not None:
            return self._rt(*args, **kw)
        return self.specialise(self.sizes_of(args))(*args, **kw)
