"""Seeded raw GGUF blocks and activations for kernel tests."""
import numpy as np

BLOCK_BYTES = {2: 18, 6: 22, 8: 34, 12: 144, 14: 210}
BLOCK_VALUES = {2: 32, 6: 32, 8: 32, 12: 256, 14: 256}
# byte offsets of the fp16 scales in a block (Q4_K: d and dmin; Q6_K: d)
SCALE_OFFSETS = {2: (0,), 6: (0,), 8: (0,), 12: (0, 2), 14: (208,)}
SPECIAL_SCALES = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x3C00, 0xBC00,
                           0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFD55, 0x1234, 0x0200],
                          np.uint16)


def f16bits(x):
    return np.asarray(x, np.float16).view(np.uint16)


def random_blocks(dtype, rows, cols, seed, special=False, scale_lo=0.002, scale_hi=0.05):
    """Raw rows of a GGUF block tensor: random codes (and K-quant sub-scales),
    fp16 scales in [scale_lo, scale_hi) with random sign (or the IEEE special
    set)."""
    rng = np.random.default_rng(seed)
    if dtype in (12, 14):
        # K-quant super-block scales multiply 6-bit (Q4_K) / int8 (Q6_K)
        # sub-scales: the same range / 64 (/ 256) gives weights of the size
        # of the 32-value formats'
        k = 64 if dtype == 12 else 256
        scale_lo, scale_hi = scale_lo / k, scale_hi / k
    nb = cols // BLOCK_VALUES[dtype]
    bb = BLOCK_BYTES[dtype]
    blk = rng.integers(0, 256, (rows, nb, bb), dtype=np.uint8)
    for off in SCALE_OFFSETS[dtype]:
        if special:
            d = SPECIAL_SCALES[rng.integers(0, SPECIAL_SCALES.size, (rows, nb))]
        else:
            d = f16bits(rng.uniform(scale_lo, scale_hi, (rows, nb)) * rng.choice([-1, 1], (rows, nb)))
        blk[:, :, off] = d & 0xFF
        blk[:, :, off + 1] = d >> 8
    return blk.reshape(rows, nb * bb)
