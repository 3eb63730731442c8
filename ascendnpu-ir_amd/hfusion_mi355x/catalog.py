"""The HFusion groups this package compiles ahead of time.

`__graft_entry__.build()` compiles each entry, so that `smoke()` and
`bench.py` on a GPU machine load prebuilt code objects: the headline
workloads of `groups.CONFIGS` at their full sizes, the bf16 and [K, N]-layout
contractions, the block-scaled fp8 contraction, the transpose+cast group, and the reduced RMSNorm+quant group
the smoke check runs.  The parity cases the tests compile (ragged sizes,
every op family of the generic lowering, dynamic dims) live beside the tests.
"""
from . import groups as g


def entries():
    """name -> IR text of every prebuilt product group."""
    e = {}
    for name, c in g.CONFIGS.items():
        e[name] = c["fn"](**c["kw"])
    e["bf16_mmad"] = g.bf16_mmad(4096, 4096, 4096)
    e["rmsnorm_quant_256"] = g.rmsnorm_quant(256, 4096)
    e["transpose_cast"] = g.transpose_cast(4096, 8192)
    # the W8A8 contraction with B in the [K, N] layout of linalg.matmul
    e["w8a8_dequant_kn"] = g.w8a8_dequant(4096, 4096, 4096, b_layout="kn").replace("@w8a8_dequant(", "@w8a8_dequant_kn(")
    # block-scaled fp8 (hfusion.matmul_mx), e4m3 x e4m3 with e8m0 scales
    e["mx_fp8"] = g.matmul_mx(4096, 4096, 4096, name="mx_fp8")
    # block-scaled fp4 (e2m1, two values per byte), 4096^3 logical
    e["mx_fp4"] = g.matmul_mx(4096, 4096, 4096, fa="e2m1", fb="e2m1", via="bitcast", name="mx_fp4")
    return e


def get(name):
    return entries()[name]
