"""NumPy statement of the bf6 block layout (srq_i4_to_bf6 in
include/signrot_hip.h), for the tests: int4 codes -> e3m2 bit fields ->
3072-byte blocks of 32 rows x 128 codes.  e3m2 (OCP MX FP6 E3M2): sign bit 5, exponent bits 4-2
(bias 3), mantissa bits 1-0; value (-1)^s 2^(e-3) (1 + m/4), or m / 16 for
e = 0."""
import numpy as np

BLOCK = 3072


def e3m2_code(c):
    """The e3m2 bit pattern of each integer in -8 .. 7."""
    c = np.asarray(c, np.int64)
    a = np.abs(c)
    e = np.where(a == 0, 0, np.floor(np.log2(np.maximum(a, 1))).astype(np.int64) + 3)
    m = np.where(a == 0, 0, (a * 4 // (1 << np.maximum(e - 3, 0))) - 4)
    return ((c < 0).astype(np.int64) << 5) | (e << 2) | m


def e3m2_value(code):
    code = np.asarray(code, np.int64)
    s = np.where(code & 32, -1.0, 1.0)
    e = (code >> 2) & 7
    m = code & 3
    return s * np.where(e == 0, m / 16.0, 2.0 ** (e - 3) * (1 + m / 4.0))


def encode(codes):
    """[R, K] int codes (K % 128 == 0) -> uint8 bf6 block layout bytes."""
    codes = np.asarray(codes, np.int64)
    R, K = codes.shape
    assert K % 128 == 0
    rp = -(-R // 32) * 32
    full = np.zeros((rp, K), np.int64)
    full[:R] = codes
    # rb, r, kb, q, h, j -> rb, kb, q, lane = r + 32 h, j
    f = e3m2_code(full).reshape(rp // 32, 32, K // 128, 2, 2, 32)
    f = f.transpose(0, 2, 3, 4, 1, 5).reshape(rp // 32, K // 128, 2, 64, 32)
    # 32 six-bit fields per lane and slice -> 24 bytes, field j at bits 6 j ..
    bits = np.zeros(f.shape[:4] + (192,), np.uint8)
    for b in range(6):
        bits[..., b::6] = (f >> b) & 1
    lb = np.packbits(bits.reshape(f.shape[:4] + (24, 8)), axis=-1, bitorder="little")
    lb = lb.reshape(f.shape[:4] + (24,))  # rb, kb, q, lane, byte
    x = lb[..., :16].reshape(f.shape[:2] + (2048,))                 # X_q at 1024 q + 16 l
    y = lb[..., 16:].transpose(0, 1, 3, 2, 4).reshape(f.shape[:2] + (1024,))  # 2048 + 16 l + 8 q
    return np.concatenate([x, y], axis=-1).reshape(-1).astype(np.uint8)


def decode(buf, R, K):
    """Inverse of encode: bf6 block layout bytes -> [R, K] int codes (the
    first R rows)."""
    buf = np.asarray(buf, np.uint8)
    rb = -(-R // 32)
    blk = buf[:rb * (K // 128) * BLOCK].reshape(rb, K // 128, BLOCK)
    x = blk[..., :2048].reshape(rb, K // 128, 2, 64, 16)
    y = blk[..., 2048:].reshape(rb, K // 128, 64, 2, 8).transpose(0, 1, 3, 2, 4)
    lb = np.concatenate([x, y], axis=-1)  # rb, kb, q, lane, 24 bytes
    bits = np.unpackbits(lb, axis=-1, bitorder="little")  # ..., 192
    f = np.zeros(lb.shape[:4] + (32,), np.int64)
    for b in range(6):
        f |= bits[..., b::6].astype(np.int64) << b
    vals = e3m2_value(f).astype(np.int64)  # rb, kb, q, lane, j
    vals = vals.reshape(rb, K // 128, 2, 2, 32, 32)  # lane = r + 32 h -> (h, r)
    codes = vals.transpose(0, 4, 1, 2, 3, 5).reshape(rb * 32, K)
    return codes[:R]
