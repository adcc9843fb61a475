"""Seeded input generators of the reference's own tests, restated in numpy.

The reference's GEMV, MoE and quantizer tests draw their inputs from SplitMix64 streams with
exactly specified float steps; restating those steps here reproduces the same inputs, so the
pinned outputs and digests the reference records check our code on identical data.
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
F = np.float32


class SplitMix:
    """splitmix64 (crates/kernels-cpu/src/gemv/tests.rs:35-45)."""

    def __init__(self, seed: int):
        self.s = seed & M64

    def next(self) -> int:
        self.s = (self.s + 0x9E3779B97F4A7C15) & M64
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)


class GemvRng(SplitMix):
    """The generator of crates/kernels-cpu/src/gemv/tests.rs:33-107."""

    def byte(self) -> int:
        return self.next() & 0xFF

    def unit(self) -> np.float32:
        # ((next >> 40) as f32 / 2^24) * 2 - 1, each step one F32 operation
        v = F(self.next() >> 40) / F(1 << 24)
        return F(F(v * F(2.0)) - F(1.0))

    def spread(self) -> np.float32:
        e = (self.next() % 13) - 6
        return F(self.unit() * F(2.0**e))

    def scale(self, f16_bits) -> bytes:
        e = (self.next() % 9) - 12
        v = F(F(F(0.5) + F(abs(self.unit()) * F(0.5))) * F(2.0**e))
        return int(f16_bits(v)).to_bytes(2, "little")


def gemv_weights(rng: GemvRng, ty: int, n_out: int, k: int, f16_bits, round_bf16) -> np.ndarray:
    """gemv/tests.rs:77-102 `weights`."""
    from oracle.oracle import BLOCK_BYTES, BLOCK_ELEMS, BF16, F16, Q4_K

    out = bytearray()
    blocks = n_out * k // BLOCK_ELEMS[ty]
    for _ in range(blocks):
        if ty == F16:
            out += int(f16_bits(rng.spread())).to_bytes(2, "little")
        elif ty == BF16:
            out += int(round_bf16(rng.spread())).to_bytes(2, "little")
        elif ty == Q4_K:
            out += rng.scale(f16_bits)
            out += rng.scale(f16_bits)
            out += bytes(rng.byte() for _ in range(4, BLOCK_BYTES[ty]))
        else:
            out += rng.scale(f16_bits)
            out += bytes(rng.byte() for _ in range(2, BLOCK_BYTES[ty]))
    return np.frombuffer(bytes(out), dtype=np.uint8).copy()


def gemv_activations(rng: GemvRng, rows: int, k: int) -> np.ndarray:
    """gemv/tests.rs:104-107."""
    return np.array([rng.spread() for _ in range(rows * k)], dtype=np.float32)


def gemv_widths(ty: int):
    """gemv/tests.rs:275-282."""
    from oracle.oracle import BF16, F16, Q4_K

    if ty in (F16, BF16):
        return [1, 7, 31, 32, 33, 64, 100, 256]
    if ty == Q4_K:
        return [256, 512, 768]
    return [32, 64, 96, 256]


# ---- crates/kernels-ggml/tests/quantize.rs:36-106 ------------------------------------------
def _pow2(e: int) -> np.float32:
    return F(2.0**e)


class QuantRng(SplitMix):
    def unit(self) -> np.float32:
        # ((next >> 40) as i32 - 2^23) as f32 * 2^-23: exact
        return F(F((self.next() >> 40) - (1 << 23)) * _pow2(-23))


TIES = [127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5, -3.5, 100.5, -100.5, 126.5, -126.5, 63.5,
        -63.5, 31.5, -31.5, 15.5, -15.5, 7.5, -7.5, 0.0, -127.0, 64.5, -64.5, 32.5, -32.5, 16.5,
        -16.5, 8.5, -8.5, 4.5]


def quant_values(seed: int, n: int) -> np.ndarray:
    """quantize.rs:66-88 `values`."""
    rng = QuantRng(seed)
    out = [F(v) for v in TIES]
    while len(out) < n:
        pick = rng.next()
        scale = _pow2((pick % 16) - 12)
        shape = (pick >> 8) % 16
        for _ in range(32):
            unit = rng.unit()
            if shape == 0:
                v = F(0.0)
            elif shape == 1:
                v = scale
            elif shape == 2 and rng.next() % 8 == 0:
                v = F(F(unit * scale) * F(64.0))
            else:
                v = F(unit * scale)
            out.append(v)
    return np.array(out[:n], dtype=np.float32)


# ---- crates/kernels-cpu/src/moe/tests.rs:40-74, 178-195 ------------------------------------
class MoeRng(SplitMix):
    def unit(self) -> np.float32:
        v = F(self.next() >> 40) / F(1 << 24)
        return F(F(v * F(2.0)) - F(1.0))

    def scale(self, f16_bits) -> bytes:
        e = (self.next() % 5) - 9
        v = F(F(F(0.5) + F(abs(self.unit()) * F(0.5))) * F(2.0**e))
        return int(f16_bits(v)).to_bytes(2, "little")


def moe_matrix(rng: MoeRng, ty: int, n_out: int, k: int, f16_bits) -> np.ndarray:
    from oracle.oracle import BLOCK_BYTES, BLOCK_ELEMS, Q4_K

    out = bytearray()
    nsc = 2 if ty == Q4_K else 1
    for _ in range(n_out * k // BLOCK_ELEMS[ty]):
        for _ in range(nsc):
            out += rng.scale(f16_bits)
        out += bytes(rng.next() & 0xFF for _ in range(2 * nsc, BLOCK_BYTES[ty]))
    return np.frombuffer(bytes(out), dtype=np.uint8).copy()


def moe_route_ids(rng: MoeRng, rows: int, top_k: int, n_experts: int) -> np.ndarray:
    ids = []
    for _ in range(rows):
        row = []
        while len(row) < top_k:
            e = rng.next() % n_experts
            if e not in row:
                row.append(e)
        ids.extend(row)
    return np.array(ids, dtype=np.int32).reshape(rows, top_k)


def moe_activations(rng: MoeRng, n: int) -> np.ndarray:
    return np.array([F(rng.unit() * F(2.0)) for _ in range(n)], dtype=np.float32)
