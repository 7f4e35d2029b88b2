"""Tile-major weight layout (include/moe_mi355x.h, moe_tiles_pack) on the host: the restated packer moves
every code word of a row exactly once, keeps each MFMA step inside one scale group, and carries each
slice's group metadata with it. The layout has no counterpart in the reference (its Metal kernels read the
state words row by row); these invariants are what the grouped kernels rely on."""
import numpy as np
import pytest
import torch

from moelab_amd import formats


def self_describing_rows(fmt, E, N, K):
    """Row records whose code word w of row n of expert e holds e << 24 | n << 12 | w + 1 (never 0), and
    whose metadata bytes hold their own position + 1 (mod 251)."""
    rb = formats.row_bytes(fmt, K)
    rows = torch.zeros((E, N, rb), dtype=torch.uint8)
    e, n, w = np.meshgrid(np.arange(E), np.arange(N), np.arange(K // 8), indexing="ij")
    words = (e << 24 | n << 12 | (w + 1)).astype(np.int32)
    rows[..., :K // 2] = torch.from_numpy(words).view(torch.uint8).reshape(E, N, K // 2)
    nmeta = K // 16 if fmt == "int4" else K // 32
    m = (np.arange(nmeta) % 251 + 1).astype(np.uint8)
    rows[..., K // 2:K // 2 + nmeta] = torch.from_numpy(np.broadcast_to(m, (E, N, nmeta)).copy())
    return rows, words


def deinterleave(w):
    """Inverse of the stored nibble order: nibble i of the stored word is element (0,2,4,6,1,3,5,7)[i]."""
    u = w.to(torch.int64) & 0xFFFFFFFF
    out = torch.zeros_like(u)
    for i, dst in enumerate((0, 2, 4, 6, 1, 3, 5, 7)):
        out |= ((u >> (4 * i)) & 0xF) << (4 * dst)
    return torch.where(out >= 2 ** 31, out - 2 ** 32, out).to(torch.int32)


def decode_pairs(w):
    """The kernels' 7-op int4 decode restated on the host: t = nibbles 0,2,4,6 and u = nibbles 1,3,5,7 in the
    low halves of bytes; the bf16 pairs are (t.b0, t.b2), (u.b0, u.b2), (t.b1, t.b3), (u.b1, u.b3). Returns the
    8 codes in the order the MFMA operand receives them."""
    t = [(w >> (8 * b)) & 0xF for b in range(4)]
    u = [(w >> (8 * b + 4)) & 0xF for b in range(4)]
    return [t[0], t[2], u[0], u[2], t[1], t[3], u[1], u[3]]


def test_stored_nibbles_decode_in_natural_order():
    """A word as stored in a tile record decodes, through the kernels' pairing, to elements 0..7 in order
    (so activations and h are used as they lie in memory)."""
    rng = np.random.default_rng(0)
    for _ in range(200):
        codes = rng.integers(0, 16, 8)
        w = int(sum(int(c) << (4 * i) for i, c in enumerate(codes)))
        w32 = torch.tensor([w - 2 ** 32 if w >= 2 ** 31 else w], dtype=torch.int32)
        stored = int(formats.interleave_nibbles(w32)[0]) & 0xFFFFFFFF
        assert decode_pairs(stored) == codes.tolist()
        assert int(deinterleave(torch.tensor([stored - 2 ** 32 if stored >= 2 ** 31 else stored],
                                             dtype=torch.int32))[0]) & 0xFFFFFFFF == w


@pytest.mark.parametrize("fmt", ["int4", "mxfp4"])
@pytest.mark.parametrize("K", [128, 192, 256, 320])
def test_every_word_moves_once_and_steps_stay_in_one_group(fmt, K):
    E, N = 2, 32
    rows, words = self_describing_rows(fmt, E, N, K)
    t = formats.pack_tiles_ref(fmt, rows, K)
    S = (K + 127) // 128
    sb = formats.TILE_SLICE_BYTES[fmt]
    nrec = E * (N // 16) * S * sb
    assert t.numel() == nrec + (E * N if fmt == "int4" else 0)   # int4: one exponent byte per row after the records
    rec = t[:nrec].reshape(E, N // 16, S, sb)
    stored = rec[..., :1024].contiguous().view(torch.int32).reshape(E, N // 16, S, 4, 16, 4)  # [.., g, r, j]
    codes = deinterleave(stored).numpy()
    nz = codes[codes != 0]
    # bijection: every (e, n, w) word exactly once, and only zero padding besides
    assert sorted(nz.tolist()) == sorted(words.reshape(-1).tolist())
    assert (codes == 0).sum() == E * (N // 16) * S * 256 - E * N * (K // 8)
    gsz = 8 if fmt == "int4" else 4   # words per scale group
    for e in range(E):
        for tile in range(N // 16):
            for s in range(S):
                for r in range(16):
                    for j in range(4):
                        ws = codes[e, tile, s, :, r, j]
                        ws = ws[ws != 0]
                        if ws.size == 0:
                            continue
                        assert np.all((ws >> 24) == e) and np.all(((ws >> 12) & 0xFFF) == 16 * tile + r)
                        widx = (ws & 0xFFF) - 1
                        # one MFMA step = one scale group, and it lies inside slice s
                        assert len(set((widx // gsz).tolist())) == 1, (s, r, j, widx)
                        assert np.all(widx // 16 == s)


@pytest.mark.parametrize("K", [128, 192])
def test_mxfp4_metadata_follows_its_slice(K):
    E, N = 1, 16
    rows, _ = self_describing_rows("mxfp4", E, N, K)
    t = formats.pack_tiles_ref("mxfp4", rows, K)
    S = (K + 127) // 128
    rec = t.reshape(E, 1, S, formats.TILE_SLICE_BYTES["mxfp4"])
    meta = rows[0, :, K // 2:].numpy()
    ng = K // 32
    for s in range(S):
        m = rec[0, 0, s, 1024:].reshape(16, 4).numpy()
        for r in range(16):
            for j in range(4):
                grp = 4 * s + j
                assert m[r, j] == (meta[r, grp] if grp < ng else 0), (s, r, j)


def int4_rows_with_meta(sc, bi, K):
    """int4 row records [1, 16, rb] with zero codes and the given bf16 scales / biases [16, K/64]."""
    rb = formats.row_bytes("int4", K)
    rows = torch.zeros((1, 16, rb), dtype=torch.uint8)
    mw = torch.stack([sc, bi], -1).contiguous().view(torch.uint8).reshape(16, K // 16)
    rows[0, :, K // 2:K // 2 + K // 16] = mw
    return rows


@pytest.mark.parametrize("K", [128, 192, 320])
def test_int4_metadata_follows_its_slice_scaled_by_the_row_exponent(K):
    """Each slice record carries its groups' (scale, bias) of each row times 2^-E_row, exactly; E_row puts the
    row's largest |s| or |b| at [2^10, 2^11); the exponent bytes follow the records. Rows span scales from 1e-30
    to 1e30 (the dense tiles' fp16 dequantisation needs the scaled values, not the raw ones, inside fp16)."""
    ng = K // 64
    rng = np.random.default_rng(K)
    mags = 10.0 ** rng.uniform(-30, 30, size=(16, 1)) * rng.uniform(0.5, 2.0, size=(16, ng))
    sc = torch.tensor(mags, dtype=torch.float32).to(torch.bfloat16)
    bi = (sc.float() * torch.tensor(rng.uniform(-12, 4, size=(16, ng)), dtype=torch.float32)).to(torch.bfloat16)
    sc[3] = 0
    bi[3] = 0                                  # an all-zero row: exponent 0
    bi[5, 0] = -sc[5, 0].float() * 300         # a row whose largest is a bias
    rows = int4_rows_with_meta(sc, bi, K)
    t = formats.pack_tiles_ref("int4", rows, K)
    S = (K + 127) // 128
    nrec = S * formats.TILE_SLICE_BYTES["int4"]
    ex = t[nrec:].view(torch.int8).to(torch.int64)
    assert ex.numel() == 16 and int(ex[3]) == 0
    amax = torch.maximum(sc.float().abs().amax(1), bi.float().abs().amax(1))
    for r in range(16):
        if r == 3:
            continue
        scaled = float(amax[r]) * 2.0 ** -int(ex[r])
        assert 1024.0 <= scaled < 2048.0, (r, float(amax[r]), int(ex[r]))
    rec = t[:nrec].reshape(S, formats.TILE_SLICE_BYTES["int4"])
    for s in range(S):
        m = rec[s, 1024:].reshape(16, 2, 2, 2).contiguous().view(torch.bfloat16)[..., 0]   # [row, group, s|b]
        for u in range(2):
            grp = 2 * s + u
            for j, src in enumerate((sc, bi)):
                got = torch.ldexp(m[:, u, j].float(), ex.float())
                want = src[:, grp].float() if grp < ng else torch.zeros(16)
                assert torch.equal(got, want), (s, u, j)


def test_int4_row_exponent_known_answers():
    """E = floor(log2 amax) - 10 from the bf16 bits: 0.16 (a bias of -8 x 0.02) -> -13; 1024 -> 0; 2047 -> 0 (bf16
    rounds it to 2048 -> 1); 1e-30 -> -110; 1e-40 (bf16 subnormal) and 1e-37 -> -120 (clamped); 3e38 -> 117;
    zero -> 0; inf and NaN -> 0."""
    vals = [0.16, 1024.0, 2047.0, 1e-30, 1e-40, 1e-37, 3e38, 0.0, float("inf"), float("nan")]
    want = [-13, 0, 1, -110, -120, -120, 117, 0, 0, 0]
    b = torch.tensor(vals, dtype=torch.float32).to(torch.bfloat16)[:, None]
    got = formats.int4_row_exponents(b, torch.zeros_like(b))
    assert got.tolist() == want
    assert formats.int4_row_exponents(torch.zeros_like(b), -b).tolist() == want   # sign ignored, bias side too
