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
    codes = rec[..., :1024].contiguous().view(torch.int32).reshape(E, N // 16, S, 4, 16, 4).numpy()  # [.., g, r, j]
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
