"""Writes tests/golden/decode_table.json: the SHA-256 of the fp32 bit patterns of every
(packed byte, scale byte) decode, element pair (even, odd), scale-major then byte.

The values come from the OCP MX E2M1 closed form and exact powers of two (Python floats),
not from the oracle's lookup table, so the digest pins the table independently. Scale bytes
>= 253 give zero with the code's sign, as lazy_lora/native/mxfp4_gemm.c:38-43 multiplies by
0.0f. When the reference's compiled C (oracle/_ref) is present the script also checks it.

    python tests/golden/make_decode_golden.py
"""
import hashlib
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))


def e2m1(code: int) -> float:
    sign = -1.0 if code & 8 else 1.0
    e, m = (code >> 1) & 3, code & 1
    mag = 0.5 * m if e == 0 else math.ldexp(1.0 + 0.5 * m, e - 1)
    return math.copysign(mag, sign)


def table() -> np.ndarray:
    out = np.empty((256, 256, 2), np.float32)
    for s in range(256):
        mult = 0.0 if s >= 253 else math.ldexp(1.0, s - 127)
        for b in range(256):
            out[s, b, 0] = np.float32(e2m1(b & 15) * mult)
            out[s, b, 1] = np.float32(e2m1(b >> 4) * mult)
    return out


def main():
    t = table()
    digest = hashlib.sha256(np.ascontiguousarray(t).view(np.uint32).tobytes()).hexdigest()
    try:
        import oracle
        ref = oracle.reference_lib()
    except Exception:
        ref = None
    if ref is not None:
        packed = np.repeat(np.arange(256, dtype=np.uint8), 16)[None, :].repeat(256, axis=0)
        scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 256, axis=1)
        got = ref.dequant(packed, scales).reshape(256, 256, 32)[:, :, :2]
        assert np.array_equal(got.view(np.uint32), t.view(np.uint32)), "reference C disagrees"
        print("reference C agrees with the closed form on all 65536 pairs")
    with open(os.path.join(HERE, "decode_table.json"), "w") as f:
        json.dump({"sha256_fp32_bits_scale_major": digest,
                   "layout": "float32 [scale 0..255][byte 0..255][even, odd] little-endian",
                   "source": "OCP MX E2M1 closed form x 2^(s-127); s >= 253 -> signed zero"}, f, indent=1)
    print(digest)


if __name__ == "__main__":
    main()
