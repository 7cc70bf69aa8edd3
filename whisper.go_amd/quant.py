"""GGUF block quantisation through libwhisper_hip.so (bit-exact with the
reference quantiser, internal/gguf/quant.go:87-248) and the device decode of
raw blocks (internal/gguf/dequant.go:47-201)."""
import ctypes as C
import os

import numpy as np

from . import native

BLOCK_BYTES = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}
BYTES_PER_WEIGHT = {0: 4.0, 1: 2.0, 2: 18 / 32, 3: 20 / 32, 6: 22 / 32, 7: 24 / 32, 8: 34 / 32}


def row_bytes(qtype, n):
    return int(native.lib().wh_row_bytes(qtype, n))


def quantize(qtype, values, threads=None):
    """Quantise a float32 array (flattened) into raw GGUF bytes of `qtype`."""
    x = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    nb = row_bytes(qtype, x.size)
    out = np.empty(nb, dtype=np.uint8)
    th = threads if threads is not None else min(16, os.cpu_count() or 1)
    native.check(native.lib().wh_quantize(qtype, x.ctypes.data, x.size, out.ctypes.data, nb, th))
    return out


def quantize_rows(qtype, mat, threads=None):
    """Quantise a [rows, cols] matrix row by row (GGUF tensors are quantised
    flat, which equals per-row quantisation when cols % 32 == 0)."""
    m = np.ascontiguousarray(mat, dtype=np.float32)
    if m.ndim != 2 or m.shape[1] % 32 == 0:
        return quantize(qtype, m, threads)
    return np.concatenate([quantize(qtype, r, threads) for r in m])


def should_quantize(name):
    return bool(native.lib().wh_should_quantize(name.encode()))


def f32_to_f16_bits(f):
    return int(native.lib().wh_f32_to_f16(float(f)))


def f16_bits_to_f32(h):
    return float(native.lib().wh_f16_to_f32(int(h)))


def dequantize_device(qtype, raw, n, device=0):
    """Decode raw GGUF blocks with the kernels' device routine (needs a GPU)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    native.check(native.lib().wh_dequantize(qtype, raw.ctypes.data, raw.size, n, out.ctypes.data, device))
    return out
