"""Comparison helpers shared by the parity tests."""
import numpy as np


def f16(bits):
    """IEEE fp16 bits -> float64 (numpy's IEEE widen)."""
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def fp16_ulp_diff(actual_bits, expected_bits):
    """Per-element |a-e| in units of the expected value's fp16 ulp, with the
    ulp floored at the smallest normal's (tests/native/vulkan/conformance-all.js:125-131)."""
    a, e = f16(actual_bits), f16(expected_bits)
    mag = np.maximum(np.abs(e), 2.0 ** -14)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 10)
    return np.abs(a - e) / ulp


def rel_err_norm(actual, expected):
    """Normwise relative error ||a-e||_2 / ||e||_2."""
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    den = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (den if den > 0 else 1.0))


def rel_err_max(actual, expected):
    """max|a-e| / max|e|."""
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    den = np.max(np.abs(e))
    return float(np.max(np.abs(a - e)) / (den if den > 0 else 1.0))


def dequant_rows(int4, scales, zp, n_rows, k):
    """Closed-form MatMulNBits dequant in float64: (q - zp) * scale,
    low nibble first, zp nibble per 32-block (even block = low nibble)."""
    b = np.asarray(int4, np.uint8).reshape(n_rows, k // 2)
    q = np.empty((n_rows, k), np.int32)
    q[:, 0::2] = b & 0xF
    q[:, 1::2] = b >> 4
    nb = k // 32
    if zp is None:
        z = np.zeros((n_rows, nb), np.int32)
    else:
        zb = np.asarray(zp, np.uint8).reshape(n_rows, -1)
        z = np.empty((n_rows, zb.shape[1] * 2), np.int32)
        z[:, 0::2] = zb & 0xF
        z[:, 1::2] = zb >> 4
        z = z[:, :nb]
    s = f16(np.asarray(scales, np.uint16).reshape(n_rows, nb))
    return (q - np.repeat(z, 32, axis=1)).astype(np.float64) * np.repeat(s, 32, axis=1)


def fp16_ieee(x):
    """float -> fp16 bits with IEEE RNE, subnormals kept (for expected values)."""
    return np.asarray(x, np.float64).astype(np.float16).view(np.uint16)
