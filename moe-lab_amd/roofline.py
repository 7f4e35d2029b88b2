"""Analytic bytes / FLOPs / floor of a SwiGLU MoE layer (expert part), priced for MI355X.

Same cost model as the reference (reference moelab/roofline.py:21-41):
    FLOPs = 6 * d * f * T * k
    bytes = U * 3 * d * f * w_bits / 8 + activations (2*T*d + 2*T*k*f) * a_bytes
    E[U]  = E * (1 - (1 - k/E)^T)
``w_bits`` counts the packed weight plus its per-group metadata: int4 g64 with a bf16 scale and a
bf16 bias per 64 weights is 4 + 32/64 = 4.5 bits; MXFP4 with one E8M0 byte per 32 weights is
4 + 8/32 = 4.25 bits. Weight-byte GB/s (the headline metric) uses only the weight term, with U
taken from the realised routing.
"""
HARDWARE = {
    # Published MI355X peaks: HBM3E 8 TB/s; dense bf16 MFMA 2.5 PFLOP/s (no sparsity).
    "mi355x": {"bw_gbs": 8000.0, "tflops_bf16": 2500.0, "label": "AMD Instinct MI355X (gfx950)"},
}

W_BITS = {"int4": 4.0 + 32.0 / 64.0, "mxfp4": 4.0 + 8.0 / 32.0, "bfloat16": 16.0, "float32": 32.0}


def expected_unique_experts(T, E, k):
    return E * (1.0 - (1.0 - k / E) ** T)


def flops(T, d, f, k, shared=0):
    return 6.0 * d * f * T * (k + shared)


def expert_bytes(d, f, fmt):
    """Packed bytes of one expert (gate + up + down), including scales/biases or E8M0 bytes."""
    return 3.0 * d * f * W_BITS[fmt] / 8.0


def weight_bytes(U, d, f, fmt, bias_bytes_per_expert=0.0, shared=0):
    return (U + shared) * (expert_bytes(d, f, fmt) + bias_bytes_per_expert)


def activation_bytes(T, d, f, k, a_bytes=2):
    return (2.0 * T * d + 2.0 * T * k * f) * a_bytes


def router_bytes(E, d, w_bytes=2):
    return float(E) * d * w_bytes


def bytes_moved(T, d, f, E, k, w_bits=16, a_bytes=2, unique=None):
    """The reference's bytes model verbatim in meaning (weights + activations)."""
    U = expected_unique_experts(T, E, k) if unique is None else unique
    return U * 3.0 * d * f * w_bits / 8.0 + activation_bytes(T, d, f, k, a_bytes)


def floor_time_s(T, d, f, E, k, hw="mi355x", w_bits=16, unique=None):
    h = HARDWARE[hw]
    t_mem = bytes_moved(T, d, f, E, k, w_bits, unique=unique) / (h["bw_gbs"] * 1e9)
    t_cmp = flops(T, d, f, k) / (h["tflops_bf16"] * 1e12)
    return max(t_mem, t_cmp)
