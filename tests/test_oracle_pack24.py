"""Pins the 2:4 packing oracle (oracle/pack24.py) — CPU only: the round trip
unpack(pack(W, M)) == W * M for 2:4 masks (bit-exact), the padding of groups
keeping fewer than two columns, the bad-group count, and the index word
layout against a direct decode of one row."""
import numpy as np

from oracle import masks as om
from oracle import pack24 as op
from oracle.numerics import round_bf16


def _case(out_f, in_f, seed):
    rng = np.random.default_rng(seed)
    W = round_bf16(rng.standard_normal((out_f, in_f)).astype(np.float32))
    M = om.hard_mask_from_soft(rng.random((out_f, in_f)).astype(np.float32), "nm_2_4")
    return W, M


def test_round_trip_two_four():
    W, M = _case(64, 128, 0)
    vals, idx, bad = op.pack(W, M)
    assert bad == 0 and vals.shape == (64, 64) and idx.shape == (2, 2, 2, 32)
    assert (op.unpack(vals, idx, 64, 128) == W * M).all()


def test_fewer_kept_are_padded_and_more_are_counted():
    W, M = _case(32, 64, 1)
    M[0, 0:4] = [0, 0, 1, 0]   # one kept
    M[1, 4:8] = 0              # none kept
    M[2, 8:12] = [1, 1, 1, 0]  # three kept: bad
    vals, idx, bad = op.pack(W, M)
    assert bad == 1
    back = op.unpack(vals, idx, 32, 64)
    assert back[0, 2] == W[0, 2] and (back[0, [0, 1, 3]] == 0).all()
    assert (back[1, 4:8] == 0).all()
    ok = np.ones(32, bool)
    ok[2] = False
    assert (back[ok] == (W * M)[ok]).all()


def test_index_word_layout_direct_decode():
    W, M = _case(32, 64, 2)
    _, idx, _ = op.pack(W, M)
    r = 5
    for sub in range(4):
        word = idx[0, 0, sub & 1, r]
        bits = (word >> (16 * (sub >> 1))) & 0xFFFF
        for grp in range(4):
            kept = [c for c in range(4) if M[r, sub * 16 + grp * 4 + c]]
            assert [(bits >> (4 * grp)) & 3, (bits >> (4 * grp + 2)) & 3] == kept


def test_tile_vals_round_trip_and_order():
    """tile_vals is a permutation (untile_vals inverts it) and puts chunk (q, kk, h) of row 32 rb + r at
    the 1 KiB run (rb, q, kk), lane h * 32 + r."""
    out_f, in_f = 64, 128
    vals = np.arange(out_f * in_f // 2, dtype=np.float32).reshape(out_f, in_f // 2)
    t = op.tile_vals(vals)
    assert np.array_equal(op.untile_vals(t), vals)
    flat = t.ravel()
    nk = in_f // 64
    for row, c16 in [(0, 0), (5, 3), (33, 6), (63, 7)]:
        rb, r, q, sub = row // 32, row % 32, c16 // 4, c16 % 4
        kk, h = sub // 2, sub % 2
        off = (((rb * nk + q) * 2 + kk) * 64 + h * 32 + r) * 8
        assert np.array_equal(flat[off:off + 8], vals[row, c16 * 8:c16 * 8 + 8])
