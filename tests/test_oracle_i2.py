"""Pins of the i2 layout oracle (oracle/i2_oracle.py), which restates
repack_signs_to_i2_cpu (patches/littlebit_cpu_optimized.cpp:712-764).

* hand-built bytes: the encoding (+1 -> 2, -1 -> 0), the group shifts, the
  byte of a column, and the dropped tail columns of a partial block;
* the reference's own op (oracle/_ref, built from the patch by
  oracle/build_ref.py) byte for byte, where it is built;
* invariants: reading the layout back gives the signs on the kept columns,
  and the kept columns are all but the tail ones counted by hand.
"""
import numpy as np
import pytest
import torch

from oracle import build_ref
from oracle import i2_oracle as I
from oracle import littlebit_oracle as O


def _words(bits_rows):
    """int32 words from rows of column bit lists (Python ints, LSB first)."""
    out = []
    for bits in bits_rows:
        nw = (len(bits) + 31) // 32
        row = []
        for w in range(nw):
            v = 0
            for j, b in enumerate(bits[32 * w:32 * w + 32]):
                v |= int(b) << j
            row.append(v - (1 << 32) if v >= 1 << 31 else v)
        out.append(row)
    return np.array(out, dtype=np.int32)


def test_four_columns_keep_only_the_first():
    # 4 columns -> 1 byte; column c sits in byte c (group 0, shift 6), so
    # columns 1-3 land in bytes 1-3 >= ceil(4/4) and are dropped
    assert I.repack_signs_to_i2(_words([[0, 0, 0, 0]]), 4).tolist() == [[0x80]]
    assert I.repack_signs_to_i2(_words([[1, 0, 0, 0]]), 4).tolist() == [[0x00]]
    assert I.repack_signs_to_i2(_words([[0, 1, 1, 1]]), 4).tolist() == [[0x80]]


def test_whole_block_all_plus_all_minus():
    assert I.repack_signs_to_i2(_words([[0] * 128]), 128).tolist() == [[0xAA] * 32]
    assert I.repack_signs_to_i2(_words([[1] * 128]), 128).tolist() == [[0x00] * 32]


def test_one_negative_column_clears_its_field():
    bits = [0] * 128
    bits[37] = 1  # group 1 (shift 4), position 5
    want = [0xAA] * 32
    want[5] = 0xAA & ~(0x3 << 4)
    assert I.repack_signs_to_i2(_words([bits]), 128).tolist() == [want]
    bits = [0] * 128
    bits[127] = 1  # group 3 (shift 0), position 31
    want = [0xAA] * 32
    want[31] = 0xA8
    assert I.repack_signs_to_i2(_words([bits]), 128).tolist() == [want]


def test_partial_block_tail():
    # 132 columns -> 33 bytes: block 1 holds columns 128-131 at group 0,
    # positions 0-3 -> bytes 32-35, of which only byte 32 exists
    out = I.repack_signs_to_i2(_words([[0] * 132]), 132)
    assert out.tolist() == [[0xAA] * 32 + [0x80]]
    # 160 columns -> 40 bytes: block 1's group 0 (columns 128-159) fills
    # bytes 32-63, of which 32-39 exist: columns 128-135 kept, 136-159 dropped
    kept = I.i2_kept_columns(160)
    assert kept[:136].all() and not kept[136:].any()


def test_pad_bits_and_extra_words_are_ignored():
    rng = np.random.default_rng(3)
    w = rng.integers(-2**31, 2**31, size=(4, 7), dtype=np.int64).astype(np.int32)
    base = I.repack_signs_to_i2(w[:, :3], 70)
    assert (I.repack_signs_to_i2(w, 70) == base).all()
    w2 = w[:, :3].copy()
    w2[:, 2] ^= np.int32(-64)  # flip bits 6-31 of the last word: columns 70-95 do not exist
    assert (I.repack_signs_to_i2(w2, 70) == base).all()


@pytest.mark.parametrize("n", [1, 4, 5, 31, 32, 33, 70, 127, 128, 129, 200, 205, 256, 298, 1843, 4096])
def test_kept_columns_read_back_as_the_signs(n):
    rng = np.random.default_rng(n)
    signs = (1 - 2 * rng.integers(0, 2, size=(5, n))).astype(np.int8)
    i2 = I.repack_signs_to_i2(O.pack_signs(signs), n)
    assert i2.shape == (5, (n + 3) // 4)
    back = I.decode_i2(i2, n)
    kept = I.i2_kept_columns(n)
    assert (back[:, kept] == signs[:, kept]).all()
    assert (back[:, ~kept] == 0).all()
    # kept: every full block of 128, then in the last block of t columns
    # the positions p < ceil(n/4) - 32 * full_blocks of each group
    full, t = divmod(n, 128)
    room = (n + 3) // 4 - 32 * full
    tail = sum(1 for c in range(t) if c % 32 < room)
    assert kept.sum() == 128 * full + tail


def test_empty():
    assert I.repack_signs_to_i2(np.zeros((0, 3), np.int32), 70).shape == (0, 18)
    assert I.repack_signs_to_i2(np.zeros((3, 0), np.int32), 0).shape == (3, 0)


@pytest.mark.skipif(not build_ref.OUT.exists(), reason="oracle/_ref not built")
@pytest.mark.parametrize("rows,n,extra", [(3, 1, 0), (3, 4, 0), (2, 70, 1), (4, 128, 0), (2, 131, 0), (3, 205, 0),
                                          (2, 298, 2), (2, 1843, 0), (2, 2686, 0), (2, 4096, 0), (2, 11008, 0)])
def test_matches_reference_op(rows, n, extra):
    ops = build_ref.load()
    rng = np.random.default_rng(100 + n)
    w = rng.integers(-2**31, 2**31, size=(rows, (n + 31) // 32 + extra), dtype=np.int64).astype(np.int32)
    ref = ops.repack_signs_to_i2(torch.from_numpy(w), n).numpy()
    assert ref.dtype == np.uint8
    assert np.array_equal(I.repack_signs_to_i2(w, n), ref)
