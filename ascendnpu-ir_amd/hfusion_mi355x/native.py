"""ctypes bindings of the two C-ABI libraries (include/hfc.h, include/hfr.h).

Nothing here falls back to another implementation: when a library is missing
the call raises, naming the file to build.
"""
import ctypes
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_ROOT, "lib")
BIN_DIR = os.path.join(PKG_ROOT, "bin")
KERNEL_INCLUDE = os.path.join(PKG_ROOT, "csrc", "kernels")

_hfc = None
_hfr = None


class NativeLibraryMissing(RuntimeError):
    pass


def _load(name):
    path = os.path.join(LIB_DIR, name)
    if not os.path.exists(path):
        raise NativeLibraryMissing(
            f"{path} is not built; run `make -C {PKG_ROOT}` (or __graft_entry__.build())")
    return ctypes.CDLL(path)


def hfc():
    """The compiler library (parse -> ConvertHFusionToHIP -> hipcc)."""
    global _hfc
    if _hfc is None:
        lib = _load("libhfc.so")
        for fn in ("hfc_compile", "hfc_compile_file"):
            f = getattr(lib, fn)
            f.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
            f.restype = ctypes.c_int
        lib.hfc_version.restype = ctypes.c_char_p
        _hfc = lib
    return _hfc


class LaunchCfg(ctypes.Structure):
    _fields_ = [("grid", ctypes.c_uint * 3), ("block", ctypes.c_uint * 3), ("lds_bytes", ctypes.c_uint)]


class GroupInfo(ctypes.Structure):
    _fields_ = [("nparams", ctypes.c_int), ("nresults", ctypes.c_int), ("nkargs", ctypes.c_int),
                ("workspace_bytes", ctypes.c_uint64), ("algo_bytes", ctypes.c_uint64),
                ("algo_ops", ctypes.c_uint64), ("cfg", LaunchCfg)]


class ProgramInfo(ctypes.Structure):
    _fields_ = [("nparams", ctypes.c_int), ("nresults", ctypes.c_int), ("nsteps", ctypes.c_int),
                ("workspace_bytes", ctypes.c_uint64)]


def hfr():
    """The runtime library (hipModuleLoad / hipModuleLaunchKernel)."""
    global _hfr
    if _hfr is None:
        lib = _load("libhfr.so")
        vp, cp = ctypes.c_void_p, ctypes.c_char_p
        lib.hfr_module_load.argtypes = [cp, ctypes.POINTER(vp)]
        lib.hfr_module_unload.argtypes = [vp]
        lib.hfr_kernel_get.argtypes = [vp, cp, ctypes.POINTER(vp)]
        lib.hfr_launch.argtypes = [vp, ctypes.POINTER(LaunchCfg), ctypes.POINTER(ctypes.c_uint64), ctypes.c_size_t, vp]
        lib.hfr_group_load.argtypes = [cp, cp, ctypes.POINTER(vp)]
        lib.hfr_group_unload.argtypes = [vp]
        lib.hfr_group_info_get.argtypes = [vp, ctypes.POINTER(GroupInfo)]
        lib.hfr_group_launch.argtypes = [vp, ctypes.POINTER(ctypes.c_uint64), ctypes.c_size_t,
                                         ctypes.POINTER(vp), ctypes.c_size_t, vp, vp]
        lib.hfr_program_load.argtypes = [cp, cp, ctypes.POINTER(vp)]
        lib.hfr_program_unload.argtypes = [vp]
        lib.hfr_program_info_get.argtypes = [vp, ctypes.POINTER(ProgramInfo)]
        lib.hfr_program_launch.argtypes = [vp, ctypes.POINTER(ctypes.c_uint64), ctypes.c_size_t,
                                           ctypes.POINTER(vp), ctypes.c_size_t, vp, vp]
        lib.hfr_group_launch_rows.argtypes = [vp, ctypes.POINTER(ctypes.c_uint64), ctypes.c_size_t,
                                              ctypes.POINTER(vp), ctypes.c_size_t, ctypes.c_int64, vp, vp]
        lib.hfr_group_launch_memref.argtypes = [vp, ctypes.POINTER(vp), ctypes.c_size_t, vp]
        lib.hfr_group_launch_noalloc.argtypes = [vp, ctypes.POINTER(ctypes.c_uint64), ctypes.c_size_t,
                                                 ctypes.POINTER(vp), ctypes.c_size_t, vp]
        lib.hfr_scratch_bytes.restype = ctypes.c_uint64
        for fn in ("hfr_module_load", "hfr_module_unload", "hfr_kernel_get", "hfr_launch", "hfr_group_load",
                   "hfr_group_unload", "hfr_group_info_get", "hfr_group_launch", "hfr_program_load",
                   "hfr_program_unload", "hfr_program_info_get", "hfr_program_launch", "hfr_group_launch_memref",
                   "hfr_group_launch_noalloc", "hfr_group_launch_rows"):
            getattr(lib, fn).restype = ctypes.c_int
        lib.hfr_last_error.restype = cp
        lib.hfr_version.restype = cp
        _hfr = lib
    return _hfr


class HfrError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"hfr error {code}: {msg}")
        self.code = code


def check(rc):
    if rc != 0:
        raise HfrError(rc, hfr().hfr_last_error().decode(errors="replace"))


def memref_descriptor(ptr, shape, offset=0, strides=None, allocated=None):
    """An MLIR ranked memref descriptor {allocated, aligned, offset,
    sizes[R], strides[R]} (the `_mlir_ciface_*` argument layout) for a buffer
    at device address `ptr`; dense row-major strides unless given."""
    rank = len(shape)
    if strides is None:
        strides, acc = [], 1
        for d in reversed(shape):
            strides.insert(0, acc)
            acc *= d

    class Desc(ctypes.Structure):
        _fields_ = [("allocated", ctypes.c_void_p), ("aligned", ctypes.c_void_p), ("offset", ctypes.c_int64),
                    ("sizes", ctypes.c_int64 * rank), ("strides", ctypes.c_int64 * rank)]

    d = Desc()
    d.allocated = ptr if allocated is None else allocated
    d.aligned = ptr
    d.offset = offset
    for i in range(rank):
        d.sizes[i] = shape[i]
        d.strides[i] = strides[i]
    return d
