"""The input generators of biv's inline kernel tests, restated so that the
oracle meets exactly the rows and activations the reference's tests use.

  rand_bytes   engine/src/quant.rs:1616-1625  (xorshift64, byte = seed >> 24)
  rand_row     engine/src/quant.rs:1627-1649  (f16 scales 0x2E66 / 0xAE66)
  ref_x        engine/src/quant.rs:1655-1657  (((i * 7919) % 211) / 50 - 2)

The kernel tests walk the types in the order Q4_0, Q4_1, Q8_0, Q4_K, Q5_K,
Q6_K on one seed; this build has no Q4_0/Q4_1/Q5_K kernels, so their rows are
drawn only to advance the seed (`advance`).
"""
import numpy as np

M64 = (1 << 64) - 1

# ggml row sizes of the types the reference tests walk through
ROW = {"Q4_0": (32, 18), "Q4_1": (32, 20), "Q8_0": (32, 34), "Q4_K": (256, 144), "Q5_K": (256, 176),
       "Q6_K": (256, 210)}
HALF = bytes.fromhex("662e")  # 0x2E66 little-endian, ~0.1
NEG = bytes.fromhex("66ae")   # 0xAE66, ~-0.1


class Seed:
    def __init__(self, v):
        self.v = v & M64


def rand_bytes(n, seed):
    out = bytearray(n)
    s = seed.v
    for i in range(n):
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        out[i] = (s >> 24) & 0xFF
    seed.v = s
    return out


def rand_row(ty, n, seed):
    be, bb = ROW[ty]
    b = rand_bytes(n // be * bb, seed)
    for o in range(0, len(b), bb):
        if ty in ("Q4_0", "Q8_0"):
            b[o:o + 2] = HALF
        elif ty == "Q4_1":
            b[o:o + 2] = HALF
            b[o + 2:o + 4] = NEG
        elif ty in ("Q4_K", "Q5_K"):
            b[o:o + 2] = HALF
            b[o + 2:o + 4] = HALF
        elif ty == "Q6_K":
            b[o + 208:o + 210] = HALF
    return np.frombuffer(bytes(b), dtype=np.uint8).copy()


def ref_x(n=1024):
    i = np.arange(n, dtype=np.int64)
    return (((i * 7919) % 211).astype(np.float32) / np.float32(50) - np.float32(2)).astype(np.float32)


def f32_sum_seq(v):
    """Sequential f32 sum (Rust's Iterator::sum over f32)."""
    s = np.float32(0)
    for a in np.asarray(v, dtype=np.float32):
        s = np.float32(s + a)
    return s
