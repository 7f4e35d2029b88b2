"""Packed expert-weight formats (host side, torch): quantise, dequantise, synthetic generation.

Both formats keep the reference's state layout (reference metal_q4_decode_v4.py:161-169,
metal_mxfp4_moe.py:448-455), so a checkpoint or a state built for the reference loads unchanged:

int4 affine, group 64 (``mx.quantize(bits=4, group_size=64)``):
    codes  [E, N, K/8]  32-bit words, 8 nibbles each, nibble i of word j <-> element 8j+i
                        (low nibble first; reference metal_q4_decode_v4.py:57-64)
    scales [E, N, K/64] bf16, biases [E, N, K/64] bf16;  w = scale * q + bias, q in [0, 15]

MXFP4 (``mx.quantize(mode="mxfp4")``):
    codes  [E, N, K/8]  32-bit words of 8 E2M1 nibbles, low nibble first
    scales [E, N, K/32] uint8 E8M0;  w = e2m1(q) * 2^(s - 127)   (reference metal_mxfp4_moe.py:1-41)
    E2M1: bit 3 = sign, bits 0..2 = magnitude index into {0, 0.5, 1, 1.5, 2, 3, 4, 6}.
    The scale byte is the float whose bit pattern is s << 23: exact 2^(s-127) for s = 1..254, 0 -> 0.

Words are held in torch.int32 tensors (same bits as the reference's uint32).

The GPU library takes each projection packed row by row (include/moe_mi355x.h): a row of K inputs is one
record of row_bytes(fmt, K) bytes = the row's K/2 code bytes followed by its group metadata (int4: one
32-bit word per group, scale bf16 in the low half, bias bf16 in the high half; MXFP4: the E8M0 bytes),
zero-padded to a multiple of 16 bytes. pack_rows / unpack_rows convert between the two layouts.
"""
import torch

GS_INT4 = 64
GS_MXFP4 = 32
E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def pack_nibbles(q):
    """q [..., K] integer codes in [0, 15] -> int32 words [..., K/8], nibble i of word j = q[8j+i]."""
    K = q.shape[-1]
    assert K % 8 == 0, K
    q = q.to(torch.int64).reshape(*q.shape[:-1], K // 8, 8)
    shifts = torch.arange(0, 32, 4, device=q.device, dtype=torch.int64)
    words = (q << shifts).sum(-1)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words)
    return words.to(torch.int32)


def unpack_nibbles(words):
    """int32 words [..., K/8] -> int64 codes [..., K]."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(0, 32, 4, device=w.device, dtype=torch.int64)
    q = (w.unsqueeze(-1) >> shifts) & 0xF
    return q.reshape(*words.shape[:-1], words.shape[-1] * 8)


# ----------------------------------------------------------------------------------- row records
FMT_INT4, FMT_MXFP4 = "int4", "mxfp4"


def row_bytes(fmt, K):
    meta = K // 16 if fmt == FMT_INT4 else K // 32
    return (K // 2 + meta + 15) // 16 * 16


def pack_rows(fmt, codes, scales, biases=None):
    """(codes int32 [E, N, K/8], scales, biases) -> uint8 records [E, N, row_bytes(fmt, K)]."""
    E, N, W = codes.shape
    K = W * 8
    rows = torch.zeros((E, N, row_bytes(fmt, K)), dtype=torch.uint8, device=codes.device)
    rows[..., :K // 2] = codes.contiguous().view(torch.uint8).reshape(E, N, K // 2)
    if fmt == FMT_INT4:
        sb = torch.stack([scales.contiguous().view(torch.int16), biases.contiguous().view(torch.int16)], dim=-1)
        rows[..., K // 2:K // 2 + K // 16] = sb.view(torch.uint8).reshape(E, N, K // 16)
    else:
        rows[..., K // 2:K // 2 + K // 32] = scales.to(torch.uint8)
    return rows


def unpack_rows(fmt, rows, K):
    """Inverse of pack_rows: (codes int32 [E, N, K/8], scales, biases) or (codes, scales) for MXFP4."""
    E, N, _ = rows.shape
    codes = rows[..., :K // 2].contiguous().view(torch.int32).reshape(E, N, K // 8)
    if fmt == FMT_INT4:
        sb = rows[..., K // 2:K // 2 + K // 16].contiguous().view(torch.int16).reshape(E, N, K // 64, 2)
        return codes, sb[..., 0].contiguous().view(torch.bfloat16), sb[..., 1].contiguous().view(torch.bfloat16)
    return codes, rows[..., K // 2:K // 2 + K // 32].contiguous()


# ------------------------------------------------------------------------------------ tile-major copy
TILE_SLICE_BYTES = {FMT_INT4: 1024 + 16 * 8, FMT_MXFP4: 1024 + 16 * 4}


def tile_word_index(fmt, s, g, j):
    """Row word (8 codes) that lane group g supplies for MFMA step j of slice s (include/moe_mi355x.h)."""
    if fmt == FMT_INT4:
        return 16 * s + 8 * (j >> 1) + 2 * g + (j & 1)
    return 16 * s + 4 * j + g


def interleave_nibbles(w):
    """int32 code words with nibbles (e0 .. e7) -> (e0, e2, e4, e6, e1, e3, e5, e7), as the tile records hold
    them (the kernels' decode pairs nibbles i and i + 4, which then are the adjacent elements 2i, 2i + 1)."""
    u = w.to(torch.int64) & 0xFFFFFFFF
    out = torch.zeros_like(u)
    for i, src in enumerate((0, 2, 4, 6, 1, 3, 5, 7)):
        out |= ((u >> (4 * src)) & 0xF) << (4 * i)
    return torch.where(out >= 2 ** 31, out - 2 ** 32, out).to(torch.int32)


def int4_row_exponents(scales, biases):
    """Row exponents of the int4 tile copies (include/moe_mi355x.h): amax = the largest bf16 magnitude over the
    row's scales and biases (bf16 [..., N, K/64] each); E = (biased exponent of amax) - 137, i.e. floor(log2
    amax) - 10, clamped to [-120, 120]; 0 for an all-zero row or one holding an inf or NaN. The records hold s 2^-E
    and b 2^-E, putting the row's largest at [2^10, 2^11)."""
    mag = lambda t: (t.contiguous().view(torch.int16).to(torch.int32) & 0x7FFF)  # noqa: E731
    amax = torch.maximum(mag(scales).amax(-1), mag(biases).amax(-1))
    ef = amax >> 7
    e = (ef - 137).clamp(-120, 120)
    return torch.where((amax == 0) | (ef >= 0xFF), torch.zeros_like(e), e)


def pack_tiles_ref(fmt, rows, K):
    """Host restatement of moe_tiles_pack: uint8 row records [E, N, row_bytes] -> uint8 [E * tile bytes].
    Test-side only (the library packs on the device); a plain loop over the documented layout. int4: the
    metadata words go in scaled by each row's 2^-E, and the E * N exponent bytes follow all the records."""
    rows = rows.cpu()
    E, N, _ = rows.shape
    S = (K + 127) // 128
    sb = TILE_SLICE_BYTES[fmt]
    words = rows[..., :K // 2].contiguous().view(torch.int32).reshape(E, N, K // 8)
    out = torch.zeros((E, N // 16, S, sb), dtype=torch.uint8)
    if fmt == FMT_INT4:
        mw = rows[..., K // 2:K // 2 + K // 16].contiguous().view(torch.int16).reshape(E, N, K // 64, 2)
        sc, bi = mw[..., 0].view(torch.bfloat16), mw[..., 1].view(torch.bfloat16)
        rexp = int4_row_exponents(sc, bi)                                   # [E, N]
        scaled = torch.stack([torch.ldexp(t.float(), -rexp[..., None].float()).to(torch.bfloat16)
                              for t in (sc, bi)], -1)                       # [E, N, K/64, 2]
        rows = rows.clone()
        rows[..., K // 2:K // 2 + K // 16] = scaled.view(torch.uint8).reshape(E, N, K // 16)
    wi = torch.tensor([[[tile_word_index(fmt, s, g, j) for j in range(4)] for g in range(4)] for s in range(S)])
    valid = wi < K // 8
    for e in range(E):
        for t in range(N // 16):
            w = words[e, 16 * t:16 * t + 16]                                  # [16 rows, K/8]
            cw = torch.where(valid[None], interleave_nibbles(w[:, wi.clamp(max=K // 8 - 1)]), 0)  # [16, S, g, j]
            out[e, t, :, :1024] = cw.permute(1, 2, 0, 3).contiguous().view(torch.uint8).reshape(S, 1024)
            meta = rows[e, 16 * t:16 * t + 16, K // 2:]
            if fmt == FMT_INT4:
                mw = meta[:, :K // 16].contiguous().view(torch.int32)        # [16, K/64]
                mw = torch.cat([mw, torch.zeros((16, 2 * S - K // 64), dtype=torch.int32)], 1)
                out[e, t, :, 1024:] = mw.reshape(16, S, 2).permute(1, 0, 2).contiguous().view(torch.uint8) \
                    .reshape(S, 128)
            else:
                mb = meta[:, :K // 32]
                mb = torch.cat([mb, torch.zeros((16, 4 * S - K // 32), dtype=torch.uint8)], 1)
                out[e, t, :, 1024:] = mb.reshape(16, S, 4).permute(1, 0, 2).reshape(S, 64)
    if fmt == FMT_INT4:
        return torch.cat([out.reshape(-1), rexp.to(torch.int8).view(torch.uint8).reshape(-1)])
    return out.reshape(-1)


# --------------------------------------------------------------------------------------------- int4
def quantize_int4(w, group_size=GS_INT4):
    """Affine 4-bit quantisation per group along the last axis, after MLX's affine quantiser:
    the group edge of larger magnitude is represented exactly (scale = edge / q0 when q0 != 0),
    scale = max((max - min) / 15, 1e-7) with the sign that maps the edge to code 0 or 15.
    Returns (codes int32 [.., K/8], scales bf16, biases bf16)."""
    *lead, K = w.shape
    assert K % group_size == 0, (K, group_size)
    wf = w.to(torch.float32).reshape(*lead, K // group_size, group_size)
    w_max = wf.amax(-1, keepdim=True)
    w_min = wf.amin(-1, keepdim=True)
    mask = w_min.abs() > w_max.abs()
    scales = torch.clamp((w_max - w_min) / 15.0, min=1e-7)
    scales = torch.where(mask, scales, -scales)
    edge = torch.where(mask, w_min, w_max)
    q0 = torch.round(edge / scales)
    scales = torch.where(q0 != 0, edge / q0, scales)
    biases = torch.where(q0 == 0, torch.zeros_like(edge), edge)
    # the kernels see bf16 scale/bias, so codes are chosen against the rounded values
    s_b = scales.to(torch.bfloat16)
    b_b = biases.to(torch.bfloat16)
    q = torch.clamp(torch.round((wf - b_b.float()) / s_b.float()), 0, 15)
    codes = pack_nibbles(q.reshape(*lead, K))
    return codes, s_b.reshape(*lead, K // group_size), b_b.reshape(*lead, K // group_size)


def dequant_int4(codes, scales, biases, group_size=GS_INT4):
    q = unpack_nibbles(codes).to(torch.float32)
    *lead, K = q.shape
    q = q.reshape(*lead, K // group_size, group_size)
    w = q * scales.float().unsqueeze(-1) + biases.float().unsqueeze(-1)
    return w.reshape(*lead, K)


def random_int4(E, N, K, generator=None, device="cpu", group_size=GS_INT4):
    """BASELINE synthetic int4 weights: uniform codes, bf16 scales ~U(0.005, 0.02), biases = -8*scale."""
    codes = random_int4_packed_words(E, N, K, generator=generator, device=device)
    scales = (torch.rand((E, N, K // group_size), generator=generator, device=device) * 0.015 + 0.005)
    scales = scales.to(torch.bfloat16)
    biases = (scales.float() * -8.0).to(torch.bfloat16)
    return codes, scales, biases


def random_int4_packed_words(E, N, K, generator=None, device="cpu"):
    """Uniform 4-bit codes drawn directly as random 32-bit words (each nibble uniform on 0..15)."""
    w = torch.randint(0, 2 ** 32, (E, N, K // 8), generator=generator, device=device,
                      dtype=torch.int64)
    return (w - (w >= 2 ** 31).to(torch.int64) * 2 ** 32).to(torch.int32)


# -------------------------------------------------------------------------------------------- MXFP4
def _e2m1_table(device):
    mags = torch.tensor(E2M1_VALUES, dtype=torch.float32, device=device)
    return torch.cat([mags, -mags])


def dequant_mxfp4(codes, scales, group_size=GS_MXFP4):
    q = unpack_nibbles(codes)
    v = _e2m1_table(q.device)[q]
    *lead, K = v.shape
    s = (scales.to(torch.int32) << 23).view(torch.float32)  # exact 2^(s-127), s = 0 -> 0
    v = v.reshape(*lead, K // group_size, group_size) * s.unsqueeze(-1)
    return v.reshape(*lead, K)


def quantize_mxfp4(w, group_size=GS_MXFP4):
    """OCP MX quantisation: per 32-group shared exponent floor(log2(amax)) - 2 (E2M1 emax = 2),
    elements rounded to the nearest E2M1 value (ties to the even code), saturating at +-6.
    Returns (codes int32 [.., K/8], scales uint8 [.., K/32])."""
    *lead, K = w.shape
    assert K % group_size == 0
    wf = w.to(torch.float32).reshape(*lead, K // group_size, group_size)
    amax = wf.abs().amax(-1, keepdim=True)
    e = torch.floor(torch.log2(torch.clamp(amax, min=2.0 ** -126))) - 2.0
    e = torch.where(amax > 0, e, torch.full_like(e, -127.0))
    sbyte = torch.clamp(e + 127.0, 0, 254)
    scale = torch.exp2(sbyte - 127.0)
    scale = torch.where(sbyte == 0, torch.ones_like(scale), scale)
    r = wf / scale
    mags = torch.tensor(E2M1_VALUES, dtype=torch.float32, device=w.device)
    a = r.abs().clamp(max=6.0).unsqueeze(-1)
    dist = (a - mags).abs()
    # ties to the even code index (E2M1's mantissa bit 0)
    best = dist.min(-1, keepdim=True).values
    cand = (dist == best)
    idx_even = torch.where(cand & (torch.arange(8, device=w.device) % 2 == 0), 1, 0)
    code_mag = torch.where(idx_even.sum(-1) > 0, (idx_even * torch.arange(8, device=w.device)).sum(-1),
                           cand.to(torch.int64).argmax(-1))
    code = code_mag + torch.where(r < 0, 8, 0) * (code_mag > 0)
    codes = pack_nibbles(code.reshape(*lead, K))
    return codes, sbyte.to(torch.uint8).reshape(*lead, K // group_size)


def random_mxfp4(E, N, K, generator=None, device="cpu", group_size=GS_MXFP4):
    """BASELINE synthetic MXFP4: uniform codes, E8M0 byte = 127 + U{-8..-4}."""
    codes = random_int4_packed_words(E, N, K, generator=generator, device=device)
    s = torch.randint(-8, -3, (E, N, K // group_size), generator=generator, device=device) + 127
    return codes, s.to(torch.uint8)
