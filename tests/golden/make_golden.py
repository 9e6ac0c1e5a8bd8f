"""Write tests/golden/int4_golden.npz: known-answer vectors for the INT4 format.

Every expected value is computed element by element in plain Python from the
definitions of the format (engine/kernels/quant.py:8-9, 115-118, 140-156):
a byte's high nibble is the even K row, its low nibble the odd K row, each a
4-bit two's complement integer, and w[k, n] = q[k, n] * scale[k // 128, n].
No vectorised code and nothing from the oracle or the product is used, so the
fixture checks both of them independently.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import random
import struct

import numpy as np

K, N, M, GROUP = 256, 64, 3, 128
HERE = os.path.dirname(os.path.abspath(__file__))


def nibble_value(v: int) -> int:
    """4-bit two's complement: 0..7 -> 0..7, 8..15 -> -8..-1."""
    return v - 16 if v >= 8 else v


def f32(v: float) -> float:
    return struct.unpack("<f", struct.pack("<f", v))[0]


def main() -> None:
    rng = random.Random(20261201)
    # Every byte value appears: the first 256 bytes (row-major) enumerate 0..255.
    data = list(range(256)) + [rng.randrange(256) for _ in range((K // 2) * N - 256)]
    packed = [[data[i * N + n] for n in range(N)] for i in range(K // 2)]
    # Varied scales per (group, column): small odd integers times powers of two.
    scale = [[f32((2 * ((g * N + n) % 7) + 1) * 2.0 ** (-(g * N + n) % 9 - 3)) for n in range(N)]
             for g in range(K // GROUP)]
    # Small integer activations keep the product exact in float32 and float64.
    x = [[float(rng.randrange(-4, 5)) for _ in range(K)] for _ in range(M)]

    q = [[0] * N for _ in range(K)]
    for i in range(K // 2):
        for n in range(N):
            b = packed[i][n]
            q[2 * i][n] = nibble_value(b >> 4)
            q[2 * i + 1][n] = nibble_value(b & 0xF)
    w = [[f32(q[k][n] * scale[k // GROUP][n]) for n in range(N)] for k in range(K)]
    y = [[0.0] * N for _ in range(M)]
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for g in range(K // GROUP):
                part = 0
                for k in range(g * GROUP, (g + 1) * GROUP):
                    part += int(x[m][k]) * q[k][n]
                acc += part * scale[g][n]
            y[m][n] = acc

    np.savez_compressed(
        os.path.join(HERE, "int4_golden.npz"),
        packed=np.array(packed, dtype=np.uint8).view(np.int8),
        scale=np.array(scale, dtype=np.float32),
        x=np.array(x, dtype=np.float32),
        codes=np.array(q, dtype=np.int8),
        dequant=np.array(w, dtype=np.float32),
        y=np.array(y, dtype=np.float64),
        group_size=np.array(GROUP),
    )


if __name__ == "__main__":
    main()
