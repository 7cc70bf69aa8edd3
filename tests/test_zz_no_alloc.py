"""wh_dequantize_noalloc (no device allocation) against wh_dequantize, through
the C ABI: bit-identical results on two calls in a row, the second with a
smaller input (the shared device array keeps the first call's contents), for
every block format; sizes past the stated maximum are rejected."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_ELEMS = 1 << 20


def _raw(wh, qtype, n, rng):
    x = (rng.standard_normal(n) * 0.5).astype(np.float32)
    if qtype == 0:
        return x.view(np.uint8).copy()
    if qtype == 1:
        return np.array([wh.quant.f32_to_f16_bits(v) for v in x[:n]], np.uint16).view(np.uint8).copy()
    return wh.quant.quantize(qtype, x)


def _noalloc(wh, qtype, raw, n):
    out = np.full(n, np.nan, np.float32)
    wh.native.check(wh.native.lib().wh_dequantize_noalloc(qtype, raw.ctypes.data, raw.size, n, out.ctypes.data, 0))
    return out


@pytest.mark.parametrize("qtype", [8, 2, 3, 6, 7, 0, 1])
def test_noalloc_matches_dequantize(wh, gpu, qtype):
    rng = np.random.default_rng(qtype + 100)
    sizes = [MAX_ELEMS, 4096 + 7] if qtype != 1 else [20000, 1000 + 3]
    for n in sizes:
        print(f"noalloc type {qtype} n {n}", flush=True)
        raw = _raw(wh, qtype, n, rng)
        want = wh.quant.dequantize_device(qtype, raw, n)
        got = _noalloc(wh, qtype, raw, n)
        assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist(), (qtype, n)


def test_noalloc_rejects_oversize(wh, gpu):
    lib = wh.native.lib()
    raw = np.zeros(wh.quant.row_bytes(8, MAX_ELEMS + 32), np.uint8)
    out = np.zeros(MAX_ELEMS + 32, np.float32)
    rc = lib.wh_dequantize_noalloc(8, raw.ctypes.data, raw.size, MAX_ELEMS + 32, out.ctypes.data, 0)
    assert rc == wh.native.WH_ERR_INVALID and b"maximum" in lib.wh_last_error()
    # short input data is an error too, not a read past the caller's buffer
    rc = lib.wh_dequantize_noalloc(8, raw.ctypes.data, 33, 64, out.ctypes.data, 0)
    assert rc == wh.native.WH_ERR_INVALID and b"short data" in lib.wh_last_error()
