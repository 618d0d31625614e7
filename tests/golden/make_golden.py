"""Writes tests/golden/known_answers.json: small known-answer vectors for the
quantized path, computed from closed forms in pure Python (integer bit
arithmetic and exact Fractions) — NOT from the oracle or the HIP library.

The reference (apepkuss/ironmlx) holds no golden vectors for quantized_matmul /
dequantize (no test touches them), and MLX itself is not available here, so
these vectors pin the stated semantics: LSB-first bit-stream packing, affine
dequant s*q+b rounded once per fp32 op then RNE to fp16, and fp32-accumulated
matmul.  Run: python tests/golden/make_golden.py
"""
import json
import os
import random
from fractions import Fraction

import numpy as np


def pack_py(codes, bits):
    acc, nbits, words = 0, 0, []
    for i, c in enumerate(codes):
        acc |= c << (i * bits)
    nwords = len(codes) * bits // 32
    return [(acc >> (32 * w)) & 0xFFFFFFFF for w in range(nwords)]


def main():
    rnd = random.Random(1234)
    out = {"pack": [], "dequant_affine": [], "qmm": []}
    for bits in (2, 3, 4, 5, 6, 8):
        codes = [rnd.randrange(1 << bits) for _ in range(64)]
        out["pack"].append({"bits": bits, "codes": codes, "words": pack_py(codes, bits)})
    for bits, gs in ((4, 32), (3, 32), (6, 64), (8, 32)):
        K = 64
        codes = [rnd.randrange(1 << bits) for _ in range(K)]
        s = np.array([rnd.uniform(-0.05, 0.05) for _ in range(K // gs)], np.float16)
        b = np.array([rnd.uniform(-0.5, 0.5) for _ in range(K // gs)], np.float16)
        res = []
        for k in range(K):
            exact = Fraction(float(s[k // gs])) * codes[k] + Fraction(float(b[k // gs]))
            # s*q is exact in fp32 (11+8 bits); the add rounds once to fp32,
            # then RNE to fp16 (numpy float32->float16 is RNE)
            v32 = np.float32(float(exact)) if abs(exact) < 2**30 else None
            # float(Fraction) is correctly rounded to double; the double->fp32
            # step equals a direct fp32 rounding unless a double tie occurs,
            # which needs > 53 bits — impossible for these 8+11+11-bit terms.
            res.append(int(np.float16(v32).view(np.uint16)))
        out["dequant_affine"].append({
            "bits": bits, "group_size": gs, "words": pack_py(codes, bits),
            "scales_f16_bits": [int(v) for v in s.view(np.uint16)],
            "biases_f16_bits": [int(v) for v in b.view(np.uint16)],
            "out_f16_bits": res})
    for bits, gs, M, N, K in ((4, 32, 2, 3, 64), (2, 64, 1, 4, 128)):
        codes = [[rnd.randrange(1 << bits) for _ in range(K)] for _ in range(N)]
        s = [[float(np.float32(rnd.uniform(-0.1, 0.1))) for _ in range(K // gs)] for _ in range(N)]
        b = [[float(np.float32(rnd.uniform(-0.1, 0.1))) for _ in range(K // gs)] for _ in range(N)]
        x = [[float(np.float32(rnd.uniform(-1, 1))) for _ in range(K)] for _ in range(M)]
        o = []
        for m in range(M):
            for n in range(N):
                acc = sum(Fraction(x[m][k]) * (Fraction(s[n][k // gs]) * codes[n][k]
                                               + Fraction(b[n][k // gs])) for k in range(K))
                o.append(float(acc))
        out["qmm"].append({"bits": bits, "group_size": gs, "M": M, "N": N,
                           "x": [v for r in x for v in r],
                           "words": [w for r in codes for w in pack_py(r, bits)],
                           "scales": [v for r in s for v in r], "biases": [v for r in b for v in r],
                           "out": o})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print("wrote", path)


if __name__ == "__main__":
    main()
