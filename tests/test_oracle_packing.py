"""Pins the oracle's bit packing (oracle/packing.py and the torch twins in oracle/attention.py).

What fixes the layout (turboquant_kv/packing.py:14-17): code d of a vector
occupies bits [d*bw, d*bw + bw) of the row read as one little-endian bit
string, LSB first; a code may straddle a byte. Checked here by

* hand-built known answers (nibble order, 3-bit and 6-bit straddles, 8-bit identity),
* brute force over every value of tiny vectors against a bit-by-bit packer
  written from that sentence alone (``_bitwise_pack`` below),
* the reference's round trip on (7, 4, 33, 128) random codes for every width
  (test_packing.py:20-40) and its byte-count KATs (test_packing.py:43-44),
* the 4-bit fast path agreeing with the general path (test_packing.py:8-17).
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import packing as opk


def _bitwise_pack(codes, bw):
    """One bit at a time: bit k of code d goes to global bit d*bw + k, byte = bit // 8."""
    nb = len(codes) * bw // 8
    out = [0] * nb
    for d, c in enumerate(codes):
        for k in range(bw):
            if (c >> k) & 1:
                g = d * bw + k
                out[g // 8] |= 1 << (g % 8)
    return out


def test_packed_bytes_kats():
    assert opk.packed_bytes(128, 3) == 48          # test_packing.py:43
    assert opk.packed_bytes(128, 4) == 64          # test_packing.py:44
    assert opk.packed_bytes(128, 6) == 96
    assert opk.packed_bytes(64, 5) == 40
    with pytest.raises(ValueError):
        opk.packed_bytes(3, 3)                      # 9 bits is not a whole byte
    assert opk.SUPPORTED == (2, 3, 4, 5, 6, 8)


def test_hand_built_vectors():
    # 4-bit: byte i = idx[2i] | idx[2i+1] << 4 (packing.py:49-54)
    assert opk.pack(np.array([[0x1, 0x2, 0xA, 0xF]], np.uint8), 4).tolist() == [[0x21, 0xFA]]
    # 3-bit: codes 5,3,6,1,7,0,2,4 -> bits 101 110 011 100 111 000 010 001 (LSB first per code)
    # global bit string (bit 0 first): 1,0,1, 1,1,0, 0,1,1, 1,0,0, 1,1,1, 0,0,0, 0,1,0, 0,0,1
    # byte0 bits0-7 = 1,0,1,1,1,0,0,1 -> 0b10011101 = 0x9D
    # byte1 bits8-15 = 1,1,0,0,1,1,1,0 -> 0b01110011 = 0x73
    # byte2 bits16-23 = 0,0,0,1,0,0,0,1 -> 0b10001000 = 0x88
    assert opk.pack(np.array([[5, 3, 6, 1, 7, 0, 2, 4]], np.uint8), 3).tolist() == [[0x9D, 0x73, 0x88]]
    # 6-bit: 0x3F, 0x01, 0x20, 0x15 -> global bits 0-5 set (code 0), bit 6 (code 1 bit 0),
    # bit 17 (code 2 bit 5), bits 18, 20, 22 (code 3 = 0b010101)
    # byte0 = bits 0-6 -> 0x7F; byte1 = 0x00; byte2 = bits 17,18,20,22 -> 2+4+16+64 = 0x56
    assert opk.pack(np.array([[0x3F, 0x01, 0x20, 0x15]], np.uint8), 6).tolist() == [[0x7F, 0x00, 0x56]]
    # 8-bit: identity
    v = np.array([[7, 200, 0, 255]], np.uint8)
    assert np.array_equal(opk.pack(v, 8), v)
    # 2-bit: 1,2,3,0 -> 0b00111001 = 0x39
    assert opk.pack(np.array([[1, 2, 3, 0]], np.uint8), 2).tolist() == [[0x39]]


@pytest.mark.parametrize("bw", [2, 3, 4, 5, 6, 8])
def test_brute_force_tiny(bw):
    """Every code value in every position of an 8-code vector, against the bitwise packer."""
    D = 8
    rows = []
    for pos, val in itertools.product(range(D), range(2 ** bw)):
        codes = [(7 * d + 3) % (2 ** bw) for d in range(D)]
        codes[pos] = val
        rows.append(codes)
    arr = np.array(rows, np.uint8)
    want = np.array([_bitwise_pack(r, bw) for r in rows], np.uint8)
    assert np.array_equal(opk.pack(arr, bw), want)
    assert np.array_equal(oa.pack_t(torch.from_numpy(arr), bw).numpy(), want)
    assert np.array_equal(opk.unpack(want, bw, D), arr)
    assert np.array_equal(oa.unpack_t(torch.from_numpy(want), bw, D).numpy(), arr)


@pytest.mark.parametrize("bw", [2, 3, 4, 5, 6, 8])
def test_round_trip_reference_shape(bw):
    """test_packing.py:20-40: (7, 4, 33, 128) random codes round-trip exactly."""
    g = torch.Generator().manual_seed(0)
    idx = torch.randint(0, 2 ** bw, (7, 4, 33, 128), dtype=torch.uint8, generator=g)
    p = opk.pack(idx.numpy(), bw)
    assert p.shape == (7, 4, 33, opk.packed_bytes(128, bw))
    assert np.array_equal(opk.unpack(p, bw, 128), idx.numpy())
    # numpy packer and the torch twin used on the oracle's hot loop agree byte for byte
    assert np.array_equal(oa.pack_t(idx, bw).numpy(), p)
    assert torch.equal(oa.unpack_t(torch.from_numpy(p), bw, 128), idx)


def test_nibble_fast_path_equals_general_path():
    """test_packing.py:8-17: the 4-bit shortcut equals the general bit path."""
    g = torch.Generator().manual_seed(1)
    idx = torch.randint(0, 16, (5, 3, 128), dtype=torch.uint8, generator=g)
    fast = oa.pack_t(idx, 4)
    sh = torch.arange(4, dtype=torch.uint8)
    bits = ((idx.reshape(-1, 128).unsqueeze(-1) >> sh) & 1).reshape(-1, 64, 8)
    general = (bits.to(torch.int16) * (1 << torch.arange(8, dtype=torch.int16))).sum(-1).to(torch.uint8)
    assert torch.equal(fast.reshape(-1, 64), general)


def test_planted_layout_mistakes_are_caught():
    """An MSB-first or byte-reversed packer fails the bitwise check (the check has teeth)."""
    codes = [5, 3, 6, 1, 7, 0, 2, 4]
    good = _bitwise_pack(codes, 3)
    msb_first = [int(f"{b:08b}"[::-1], 2) for b in good]
    assert msb_first != good
    assert good[::-1] != good
    assert opk.pack(np.array([codes], np.uint8), 3).tolist() == [good]
