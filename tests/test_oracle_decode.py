"""Pins the oracle's MXFP4 decode (mxfp4_gemm.c:30-62, :142-150) without trusting its own table:
against the OCP E2M1 closed form, the reference's compiled C, the committed golden digest of
all 65,536 (byte, scale) pairs, and the special cases the reference documents."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "decode_table.json")


def exhaustive_pairs():
    """Every packed byte against every scale byte. Row s uses scale s for all its blocks;
    block b of a row is byte value b repeated 16 times. packed [256, 4096], scales [256, 256]."""
    packed = np.repeat(np.arange(256, dtype=np.uint8), 16)[None, :].repeat(256, axis=0)
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 256, axis=1)
    return packed, scales


def test_e2m1_table_matches_closed_form():
    for code in range(16):
        want = oracle.e2m1_closed_form(code)
        assert np.float32(want).view(np.uint32) == oracle.E2M1[code].view(np.uint32), code
    # code 8 is negative zero (mxfp4_gemm.c:33-34)
    assert oracle.E2M1[8].view(np.uint32) == 0x80000000


def test_e8m0_table():
    t = oracle.e8m0_table()
    for s in range(253):
        assert float(t[s]) == 2.0 ** (s - 127), s
    assert t[0].view(np.uint32) == 0x00400000  # 2^-127 is an fp32 subnormal
    assert np.all(t[253:] == 0)


def test_dequant_closed_form_every_pair():
    packed, scales = exhaustive_pairs()
    got = oracle.dequant(packed, scales)  # [256 scales, 256 bytes * 32]
    got = got.reshape(256, 256, 32)
    for s in (0, 1, 2, 64, 126, 127, 128, 200, 250, 252, 253, 254, 255):
        mult = 0.0 if s >= 253 else 2.0 ** (s - 127)
        for byte in range(256):
            lo = np.float32(oracle.e2m1_closed_form(byte & 15) * mult)
            hi = np.float32(oracle.e2m1_closed_form(byte >> 4) * mult)
            assert got[s, byte, 0].view(np.uint32) == lo.view(np.uint32), (s, byte)
            assert got[s, byte, 1].view(np.uint32) == hi.view(np.uint32), (s, byte)


def test_dequant_golden_digest():
    """SHA-256 of the fp32 bits of all 65,536 (byte, scale) decodes, committed as a fixture."""
    packed, scales = exhaustive_pairs()
    got = oracle.dequant(packed, scales).reshape(256, 256, 32)[:, :, :2]
    digest = hashlib.sha256(np.ascontiguousarray(got).view(np.uint32).tobytes()).hexdigest()
    with open(GOLDEN) as f:
        want = json.load(f)["sha256_fp32_bits_scale_major"]
    assert digest == want


def test_dequant_matches_reference_c(reflib, clib):
    packed, scales = exhaustive_pairs()
    a = oracle.dequant(packed, scales)
    b = reflib.dequant(packed, scales)
    c = clib.dequant(packed, scales)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(c.view(np.uint32), b.view(np.uint32))


def test_special_values():
    # damaged scale bytes contribute signed zeros, never inf/NaN (mxfp4_gemm.c:16-18, :41)
    packed = np.array([[0x98] * 16], np.uint8)  # codes 8 (-0.0) and 9 (-0.5)
    for s in (253, 254, 255):
        w = oracle.dequant(packed, np.array([[s]], np.uint8))
        assert np.all(w == 0) and np.all(np.signbit(w)), s
    # scale byte 0 and 1 give fp32 subnormals
    w = oracle.dequant(np.array([[0x71] * 16], np.uint8), np.array([[0]], np.uint8))
    assert w[0, 0] == np.float32(2.0 ** -128) and w[0, 1] == np.float32(6 * 2.0 ** -127)
    assert 0 < w[0, 0] < np.finfo(np.float32).tiny
