"""The oracle's f16 / dequantisation / quantiser restatements pinned against the
reference's known-answer tests (internal/gguf/gguf_test.go:155-309,
quant_test.go:11-127), an exhaustive IEEE check and an independent numpy
restatement; and the product's host quantiser bit-exact against the oracle."""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
QTYPES = [2, 3, 6, 7, 8]


def test_f16_kats(orc, wh):
    for k in json.load(open(os.path.join(GOLDEN, "f16_kats.json"))):
        want = int(k["f32_bits"], 16)
        assert np.float32(orc.f16_to_f32(k["h"])).view(np.uint32) == want, k["name"]
        assert np.float32(wh.quant.f16_bits_to_f32(k["h"])).view(np.uint32) == want, k["name"]
    assert np.isnan(orc.f16_to_f32(0x7E00))


def test_f16_decode_exhaustive(orc, wh):
    """Every f16 pattern: the decode equals IEEE binary16 -> binary32 (numpy),
    NaN payloads kept as the reference does (sign | 0x7F800000 | m << 13)."""
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32).view(np.uint32).copy()
    nan = ((h >> 10) & 0x1F) == 31
    ref[nan] = ((h[nan].astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | ((h[nan].astype(np.uint32) & 0x3FF) << 13)
    # through a float32 buffer (a C float return value would quiet signalling NaNs)
    got_o = orc.dequantize(h.view(np.uint8), 1, h.size).view(np.uint32)
    assert np.array_equal(got_o, ref)
    quiet = ~nan | ((h & 0x200) != 0)
    sel = np.nonzero(quiet)[0][::7]
    got_p = np.array([wh.quant.f16_bits_to_f32(int(v)) for v in h[sel]], np.float32).view(np.uint32)
    assert np.array_equal(got_p, ref[sel])


def test_dequant_kats(orc):
    for k in json.load(open(os.path.join(GOLDEN, "dequant_kats.json"))):
        out = orc.dequantize(np.array(k["block"], np.uint8), k["type"], 32)
        for i, v in k["expect"].items():
            assert out[int(i)] == np.float32(v), (k["name"], i)


def _np_f32_to_f16_halfup(x):
    """Independent numpy restatement of gguf/quant.go:11-55 (round half-up on
    mantissa bit 12, f32 subnormals -> signed zero)."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.int64)
    sign = (b >> 31) << 15
    exp = (b >> 23) & 0xFF
    mant = b & 0x7FFFFF
    e16 = exp - 112
    m16 = (mant >> 13) + ((mant >> 12) & 1)
    carry = m16 >= 0x400
    m16 = np.where(carry, 0, m16)
    e16c = np.where(carry, e16 + 1, e16)
    normal = sign | (e16c << 10) | m16
    sub = sign | ((mant | 0x800000) >> np.clip(14 - e16, 0, 63))
    out = np.where(e16c >= 31, sign | 0x7C00, normal)
    out = np.where(e16 <= 0, np.where(e16 < -10, sign, sub), out)
    out = np.where(exp == 0, sign, out)
    out = np.where(exp == 255, np.where(mant != 0, sign | 0x7E00, sign | 0x7C00), out)
    return out.astype(np.uint16)


def _np_round_half_away(v):
    return np.where(v >= 0, np.floor(v.astype(np.float64) + 0.5), -np.floor(-v.astype(np.float64) + 0.5))


def _np_quant_q8_0(x):
    """numpy restatement of QuantizeQ8_0 (quant.go:202-232) for n % 32 == 0."""
    blk = x.reshape(-1, 32).astype(np.float32)
    scale = (np.max(np.abs(blk), axis=1) / np.float32(127.0)).astype(np.float32)
    q = np.zeros_like(blk, dtype=np.int64)
    nz = scale != 0
    q[nz] = np.clip(_np_round_half_away((blk[nz] / scale[nz, None]).astype(np.float32)), -127, 127)
    out = np.zeros((blk.shape[0], 34), np.uint8)
    h = _np_f32_to_f16_halfup(scale)
    out[:, 0] = h & 0xFF
    out[:, 1] = h >> 8
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def test_f32_to_f16_vs_numpy_restatement(orc, wh):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-9, 5, 20000),
                        np.array([0.0, -0.0, 65504, 65520, 1e6, -1e6, 6e-8, 6.1e-5, 5.96e-8, 2.98e-8, 1e-40,
                                  np.inf, -np.inf], np.float32)]).astype(np.float32)
    want = _np_f32_to_f16_halfup(x)
    got = np.array([orc.f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)
    got_p = np.array([wh.quant.f32_to_f16_bits(float(v)) for v in x[::5]], np.uint16)
    assert np.array_equal(got_p, want[::5])


def test_f16_conversion_roundtrips(orc):
    """quant_test.go:88-127."""
    cases = [(0.0, 0), (1.0, 0), (-1.0, 0), (0.5, 0), (65504.0, 0), (float(np.float32(2.0 ** -24)), 1e-30)]
    for f, tol in cases:
        got = orc.f16_to_f32(orc.f32_to_f16(f))
        t = tol or max(abs(f) * 1e-3, 1e-6)
        assert abs(got - f) <= t


def test_quantize_q8_0_vs_numpy_restatement(orc, wh):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(32 * 4000) * 0.02).astype(np.float32)
    x[:64] = 0.0
    x[64:96] = 0.37
    x[96:128] = np.linspace(-1, 1, 32)
    want = _np_quant_q8_0(x)
    assert orc.quantize(x, 8).tobytes() == want.tobytes()
    assert wh.quant.quantize(8, x).tobytes() == want.tobytes()


@pytest.mark.parametrize("qtype", [1] + QTYPES)
def test_product_quantizer_bit_exact(orc, wh, qtype):
    rng = np.random.default_rng(qtype)
    for n in (1, 7, 31, 32, 33, 1000, 32 * 513):
        for scale in (0.02, 1.0, 3e4, 1e-7):
            x = (rng.standard_normal(n) * scale).astype(np.float32)
            if n >= 32:
                x[:32] = x[0]          # constant block (zero range)
            if n >= 64:
                x[32:64] = 0.0         # all-zero block
            a = wh.quant.quantize(qtype, x)
            b = orc.quantize(x, qtype)
            assert a.tobytes() == b.tobytes(), (qtype, n, scale)


@pytest.mark.parametrize("qtype,tol", [(2, 0.1), (3, 0.1), (6, 0.05), (7, 0.05), (8, 0.01), (1, 0.001)])
def test_quant_roundtrip_bounds(orc, qtype, tol):
    """quant_test.go:11-85: the ramp -1..1 over one block."""
    x = (np.arange(32, dtype=np.float32) / np.float32(31) * 2 - 1).astype(np.float32)
    back = orc.dequantize(orc.quantize(x, qtype), qtype, 32)
    assert np.max(np.abs(back - x)) <= tol


def test_quantizer_invariants(orc):
    """Closed-form invariants: Q8_0 scale word = f16(absmax/127) and |q| <= 127;
    Q4/Q5 interleaving (element 2i = low nibble, 2i+1 = high nibble; qh bit j
    = element j's fifth bit); Q4_1/Q5_1 min word = f16(min)."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32) * 0.5).astype(np.float32)
    q8 = orc.quantize(x, 8)
    amax = np.float32(np.max(np.abs(x)))
    assert int(q8[0]) | int(q8[1]) << 8 == orc.f32_to_f16(float(amax / np.float32(127)))
    codes = q8[2:].view(np.int8).astype(int)
    assert np.all(np.abs(codes) <= 127) and np.max(np.abs(codes)) == 127
    q4 = orc.quantize(x, 2)
    d = amax / np.float32(7.0)
    for i in range(32):
        nib = (q4[2 + i // 2] >> (4 * (i & 1))) & 0xF
        assert nib == np.clip(_np_round_half_away(np.array([x[i] / d], np.float32))[0] + 8, 0, 15)
    q5 = orc.quantize(x, 7)
    mn = np.float32(np.min(x))
    assert int(q5[2]) | int(q5[3]) << 8 == orc.f32_to_f16(float(mn))
    qh = int.from_bytes(q5[4:8].tobytes(), "little")
    d5 = (np.float32(np.max(x)) - mn) / np.float32(31.0)
    for i in range(32):
        code = int(_np_round_half_away(np.array([(x[i] - mn) / d5], np.float32))[0])
        code = min(max(code, 0), 31)
        nib = (q5[8 + i // 2] >> (4 * (i & 1))) & 0xF
        assert nib == code & 0xF and ((qh >> i) & 1) == code >> 4


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_closed_form(orc, qtype):
    """dequant = d*q (+ m) computed independently in numpy from the block fields."""
    rng = np.random.default_rng(10 + qtype)
    raw = rng.integers(0, 256, size=64 * {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}[qtype], dtype=np.uint8)
    bb = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}[qtype]
    for b in range(64):  # finite scales
        raw[b * bb + 1] &= 0x3F
        if qtype in (3, 7):
            raw[b * bb + 3] &= 0x3F
    got = orc.dequantize(raw, qtype, 64 * 32)
    blocks = raw.reshape(64, bb)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    if qtype == 8:
        q = blocks[:, 2:].view(np.int8).astype(np.float32)
        want = d[:, None] * q
    else:
        off = {2: 2, 3: 4, 6: 6, 7: 8}[qtype]
        qs = blocks[:, off:off + 16]
        lo, hi = (qs & 0xF).astype(np.int64), (qs >> 4).astype(np.int64)
        nib = np.empty((64, 32), np.int64)
        nib[:, 0::2], nib[:, 1::2] = lo, hi
        if qtype in (6, 7):
            hb = blocks[:, 2 if qtype == 6 else 4:(2 if qtype == 6 else 4) + 4].copy().view(np.uint32).reshape(-1)
            nib |= ((hb[:, None] >> np.arange(32)) & 1).astype(np.int64) << 4
        if qtype in (2, 6):
            want = d[:, None] * (nib - (8 if qtype == 2 else 16)).astype(np.float32)
        else:
            m = blocks[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(-1)
            want = (d[:, None] * nib.astype(np.float32)).astype(np.float32) + m[:, None]
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).reshape(-1).view(np.uint32))


def test_should_quantize_rule(orc, wh):
    """P5 (gguf/quant.go:236-248): per-block LN gains are quantised, decoder.ln,
    biases and the positional embedding are not."""
    cases = {
        "decoder.token_embedding.weight": True, "decoder.positional_embedding": False,
        "decoder.blocks.0.self_attn_ln.weight": True, "decoder.blocks.0.cross_attn_ln.weight": True,
        "decoder.blocks.3.mlp_ln.weight": True, "decoder.blocks.3.mlp_ln.bias": False,
        "decoder.ln.weight": False, "decoder.ln.bias": False, "decoder.blocks.0.mlp.0.weight": True,
        "decoder.blocks.0.mlp.0.bias": False, "encoder.blocks.0.attn_ln.weight": True,
        "model.decoder.layer_norm.weight": False, "X.NORM.weight": False,
    }
    for name, want in cases.items():
        assert orc.should_quantize(name) == want, name
        assert wh.quant.should_quantize(name) == want, name
