"""moelab_amd: MI355X-native (gfx950) quantised MoE-layer hot path of Tigerly1/moe-lab.

Host code in Python on PyTorch-ROCm; GPU work in hand-written HIP kernels behind the C ABI of
libmoe_mi355x.so (include/moe_mi355x.h). The directory is named ``moe-lab_amd``; it is imported as
``moelab_amd`` (see __graft_entry__.load_package).

Modules:
    shapes, roofline, problem   spec: shapes, cost model, seeded inputs and BASELINE configs
    formats                     int4 g64 / MXFP4 packing (reference state layouts)
    router                      fused gate GEMV + router tail, stable slot grouping
    experts, fallback           the expert-path call and the per-slot stock-style path
    variants/                   drop-in variant modules (prepare / run / dequant contract)
    backend                     torch-ROCm harness: fp32 reference, errors, chained timing
"""
__version__ = "0.1.0"
