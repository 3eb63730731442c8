"""MI355X-native backend for BiShengIR HFusion op groups.

    import hfusion_mi355x as hf
    grp = hf.load(hf.groups.vec_add(1 << 24))   # bishengir-compile + load
    out = grp(a, b, out)                         # launch on the current stream

The compile step is `bishengir-compile --target=mi355x` (libhfc); the launch
goes through the C-ABI runtime libhfr (hipModuleLaunchKernel).
"""
from . import catalog, groups, inputs, native
from .runtime import Artifact, CompileError, DynamicGroup, Group, Program, compile, load, parse_manifest, torch_dtype

__all__ = ["Artifact", "CompileError", "DynamicGroup", "Group", "catalog", "compile", "groups", "inputs", "load", "native",
           "parse_manifest", "torch_dtype", "Program"]
