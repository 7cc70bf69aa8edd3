"""C-ABI surface and host logic (no GPU needed)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "whisper_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(wh):
    lib = wh.native.lib()
    syms = declared_symbols()
    assert len(syms) >= 30
    for s in syms:
        assert hasattr(lib, s), s
    assert sorted(wh.native.EXPORTED) == syms


def test_version_and_sizes(wh):
    lib = wh.native.lib()
    assert b"gfx950" in lib.wh_version()
    for t, per in [(8, 34), (2, 18), (3, 20), (6, 22), (7, 24)]:
        assert lib.wh_row_bytes(t, 1280) == 40 * per
        assert lib.wh_row_bytes(t, 33) == 2 * per
    assert lib.wh_row_bytes(0, 10) == 40 and lib.wh_row_bytes(1, 10) == 20
    assert lib.wh_row_bytes(12, 256) == 0


def test_error_paths(wh):
    lib = wh.native.lib()
    h = C.c_void_p()
    raw = np.zeros(10, np.uint8)
    rc = lib.wh_matrix_create(8, 0, 32, raw.ctypes.data, raw.size, 0, C.byref(h))
    assert rc == wh.native.WH_ERR_INVALID and b"invalid dims" in lib.wh_last_error()
    rc = lib.wh_matrix_create(8, 2, 64, raw.ctypes.data, raw.size, 0, C.byref(h))
    assert rc == wh.native.WH_ERR_INVALID and b"short data" in lib.wh_last_error()
    rc = lib.wh_matrix_create(12, 2, 64, raw.ctypes.data, raw.size, 0, C.byref(h))
    assert rc == wh.native.WH_ERR_UNSUPPORTED
    x = np.zeros(64, np.float32)
    out = np.zeros(10, np.uint8)
    assert lib.wh_quantize(8, x.ctypes.data, 64, out.ctypes.data, out.size, 1) == wh.native.WH_ERR_INVALID
    assert lib.wh_quantize(12, x.ctypes.data, 64, out.ctypes.data, out.size, 1) == wh.native.WH_ERR_UNSUPPORTED
    assert lib.wh_model_hparams(None, None) == wh.native.WH_ERR_INVALID
    assert lib.wh_model_load_gguf(b"/nonexistent.gguf", 0, C.byref(h)) == wh.native.WH_ERR_INVALID
    assert b"gguf: open" in lib.wh_last_error()


def test_error_message_is_thread_local(wh):
    import threading

    lib = wh.native.lib()
    h = C.c_void_p()
    raw = np.zeros(1, np.uint8)
    lib.wh_matrix_create(8, 0, 32, raw.ctypes.data, 1, 0, C.byref(h))
    seen = []

    def other():
        seen.append(lib.wh_last_error())

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen == [b""] and b"invalid dims" in lib.wh_last_error()


def test_quantizer_threads_do_not_change_bytes(wh):
    x = np.random.default_rng(0).standard_normal(32 * 50000).astype(np.float32)
    for qt in (2, 3, 6, 7, 8):
        assert wh.quant.quantize(qt, x, threads=1).tobytes() == wh.quant.quantize(qt, x, threads=8).tobytes()


def test_synthetic_decoder_layout(wh):
    """Names and shapes of internal/model/decoder.go:176-296; quantisation by
    the cmd/quantize rule; each tensor seeded independently."""
    tensors, meta = wh.synth.make_decoder("layout", 8, dims=(500, 64, 1, 2, 16))
    by = {t.name: t for t in tensors}
    assert len(tensors) == 2 + 2 * 24 + 2
    assert by["decoder.token_embedding.weight"].shape == (500, 64) and by["decoder.token_embedding.weight"].type == 8
    assert by["decoder.positional_embedding"].type == 0
    assert by["decoder.blocks.1.mlp.0.weight"].shape == (256, 64)
    assert by["decoder.blocks.1.mlp.2.weight"].shape == (64, 256)
    assert by["decoder.blocks.0.self_attn_ln.weight"].type == 8   # P5: quantised LN gain
    assert by["decoder.ln.weight"].type == 0 and by["decoder.blocks.0.mlp.0.bias"].type == 0
    g = np.frombuffer(by["decoder.ln.weight"].data.tobytes(), np.float32)
    assert abs(g.mean() - 1) < 0.01 and 0.01 < g.std() < 0.03
    again, _ = wh.synth.make_decoder("layout", 8, dims=(500, 64, 1, 2, 16))
    assert all(a.data.tobytes() == b.data.tobytes() for a, b in zip(tensors, again))
    other, _ = wh.synth.make_decoder("layout2", 8, dims=(500, 64, 1, 2, 16))
    assert tensors[0].data.tobytes() != other[0].data.tobytes()


def _bytes_from_shapes(config, qtype):
    V, d, H, L, ctx = wh_configs()[config]
    per = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}[qtype]
    return (14 * d * d * L + V * d) // 32 * per


def wh_configs():
    import __graft_entry__

    return __graft_entry__.load_package().synth.CONFIGS


@pytest.mark.parametrize("config,qtype,want", [("large-v3", 8, 850416160), ("tiny.en", 8, 29934144),
                                                ("small", 7, 104191488), ("large-v3", 3, 500244800)])
def test_weight_bytes_per_token(config, qtype, want):
    """Algorithmic weight bytes per decode step (14 d^2 per layer + V d)."""
    assert _bytes_from_shapes(config, qtype) == want


def test_weight_bytes_helper_matches_formula(wh):
    tensors, meta = wh.synth.make_decoder("wb", 8, dims=(1000, 128, 2, 3, 16))
    assert wh.synth.weight_bytes_per_token(tensors) == (14 * 128 * 128 * 3 + 1000 * 128) // 32 * 34


def test_gguf_roundtrip(wh, tmp_path):
    tensors, meta = wh.synth.make_decoder("gguf", 7, dims=(300, 64, 1, 1, 16))
    path = str(tmp_path / "m.gguf")
    wh.synth.write_gguf(path, tensors, meta)
    raw = open(path, "rb").read()
    assert raw[:4] == b"GGUF" and int.from_bytes(raw[4:8], "little") == 3
    back, m2 = wh.synth.read_gguf(path)
    assert m2["whisper.decoder.embedding_length"] == 64 and m2["whisper.vocab.size"] == 300
    assert [t.name for t in back] == [t.name for t in tensors]
    for a, b in zip(tensors, back):
        assert a.type == b.type and a.shape == b.shape and a.data.tobytes() == b.data.tobytes()


def test_decoder_params_defaults(wh):
    p = wh.DecoderParams()
    assert p.prompt == [] and p.beam_size == 0 and p.temperature == 0.0 and not p.no_fallback


def test_gguf_parse_errors(wh, tmp_path):
    """internal/gguf/gguf.go:69-135: bad magic, unsupported version and a
    truncated header fail before any device work."""
    lib = wh.native.lib()
    h = C.c_void_p()
    cases = {
        "magic": b"GGUX" + b"\0" * 28,
        "version": b"GGUF" + (7).to_bytes(4, "little") + b"\0" * 24,
        "truncated": b"GGUF" + (3).to_bytes(4, "little") + (1).to_bytes(8, "little") + (5).to_bytes(8, "little")
        + b"\x05\0\0\0\0\0\0\0abc",
    }
    want = {"magic": (wh.native.WH_ERR_INVALID, b"invalid magic"),
            "version": (wh.native.WH_ERR_UNSUPPORTED, b"unsupported version"),
            "truncated": (wh.native.WH_ERR_INVALID, b"truncated")}
    for name, blob in cases.items():
        path = tmp_path / f"{name}.gguf"
        path.write_bytes(blob)
        rc = lib.wh_model_load_gguf(str(path).encode(), 0, C.byref(h))
        assert (rc, want[name][1] in lib.wh_last_error()) == (want[name][0], True), name
