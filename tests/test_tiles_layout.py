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
    assert t.numel() == E * (N // 16) * S * sb
    rec = t.reshape(E, N // 16, S, sb)
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


@pytest.mark.parametrize("fmt", ["int4", "mxfp4"])
@pytest.mark.parametrize("K", [128, 192])
def test_metadata_follows_its_slice(fmt, K):
    E, N = 1, 16
    rows, _ = self_describing_rows(fmt, E, N, K)
    t = formats.pack_tiles_ref(fmt, rows, K)
    S = (K + 127) // 128
    rec = t.reshape(E, 1, S, formats.TILE_SLICE_BYTES[fmt])
    meta = rows[0, :, K // 2:].numpy()
    if fmt == "int4":
        ng = K // 64
        for s in range(S):
            m = rec[0, 0, s, 1024:].reshape(16, 2, 4).numpy()
            for r in range(16):
                for u in range(2):
                    grp = 2 * s + u
                    want = meta[r, 4 * grp:4 * grp + 4] if grp < ng else np.zeros(4, np.uint8)
                    assert np.array_equal(m[r, u], want), (s, r, u)
    else:
        ng = K // 32
        for s in range(S):
            m = rec[0, 0, s, 1024:].reshape(16, 4).numpy()
            for r in range(16):
                for j in range(4):
                    grp = 4 * s + j
                    assert m[r, j] == (meta[r, grp] if grp < ng else 0), (s, r, j)
