"""The device encoder (internal/model/encoder.go:58-396) through the C ABI
against the oracle's encoder on the same seeded weights and log-mel input.

Bar: max |device - oracle| within 2e-4 of max |oracle| (the products sum in
another order on the matrix cores; the softmax is the reference's fast exp on
both sides). Covers quantised and float weights, head size 64 (the tiled
attention kernel) and another head size (the generic one), odd frame counts,
the stored weight orders and HF names the reference accepts, GGUF files with
and without metadata, the frame-count rules, cancellation, the full-size
tiny.en encoder, the large-v3 shapes over a full window, and mel -> encoder ->
decoder tokens end to end.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = 2e-4


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


ENC_MODELS = [
    # name, qtype, (n_mels, d, heads, layers, n_ctx), T
    ("eq8", 8, (16, 128, 2, 2, 100), 200),
    ("eq41", 3, (16, 256, 4, 2, 150), 299),
    ("eq51", 7, (24, 192, 3, 1, 130), 260),
    ("ef32", 0, (16, 128, 2, 1, 70), 139),
    ("ehd32", 8, (16, 128, 4, 2, 80), 160),  # head size 32: the generic attention kernel
]


@pytest.mark.parametrize("name,qtype,dims,T", ENC_MODELS)
def test_encoder_vs_oracle(wh, orc, gpu, name, qtype, dims, T):
    print(f"encoder {name} T={T}", flush=True)
    tensors, meta = wh.synth.make_encoder(name, qtype, dims=dims)
    mel = wh.synth.mel_input(name, dims[0], T=T)
    enc = wh.HIPEncoder(tensors, meta)
    assert (enc.n_mels, enc.n_state, enc.n_head, enc.n_layer, enc.n_ctx) == dims
    got = enc.encode(mel)
    want = orc.OracleEncoder(tensors, meta, threads=8).encode(mel)
    assert got.shape == want.shape == ((T + 1) // 2, dims[1])
    assert _rel(got, want) < TOL, (name, _rel(got, want))
    # a second call on the same handle gives the same bits
    assert np.array_equal(enc.encode(mel), got)
    enc.close()


def test_encoder_layouts_and_names(wh, orc, gpu):
    """The legacy [n_mels, d, 3] conv1 order, a [3, d, d] conv2, a [d, n_ctx]
    positional embedding and the HF names load to the same encoder
    (encoder.go:121-185, compat.go:31-83); without metadata the sizes are
    inferred (head count d / 64)."""
    dims = (16, 128, 2, 1, 60)
    tensors, meta = wh.synth.make_encoder("elay", 0, dims=dims)
    mel = wh.synth.mel_input("elay", 16, T=120)
    base = wh.HIPEncoder(tensors, meta)
    want = base.encode(mel)
    base.close()
    alt = []
    for t in tensors:
        x = t.data.view(np.float32).reshape(t.shape)
        if t.name == "encoder.conv1.weight":
            alt.append(wh.synth.Tensor("model.encoder.conv1.weight", 0, (16, 128, 3),
                                       np.ascontiguousarray(x.transpose(1, 0, 2))))
        elif t.name == "encoder.conv2.weight":
            alt.append(wh.synth.Tensor(t.name, 0, (3, 128, 128), np.ascontiguousarray(x.transpose(2, 1, 0))))
        elif t.name == "encoder.positional_embedding":
            alt.append(wh.synth.Tensor(t.name, 0, (128, 60), np.ascontiguousarray(x.T)))
        elif t.name == "encoder.blocks.0.attn.query.weight":
            alt.append(wh.synth.Tensor("model.encoder.layers.0.self_attn.q_proj.weight", 0, t.shape, x))
        else:
            alt.append(t)
    enc = wh.HIPEncoder(alt, None)
    assert (enc.n_mels, enc.n_state, enc.n_head, enc.n_layer, enc.n_ctx) == dims
    assert _rel(enc.encode(mel), want) < 1e-6
    enc.close()


def test_encoder_frame_rules(wh, orc, gpu):
    """T = 2 n_ctx + 1 keeps the first n_mels * 2 n_ctx values of the buffer (as
    the reference re-slices it); T > 2 n_ctx and a wrong band count are errors."""
    tensors, meta = wh.synth.make_encoder("efr", 8, dims=(16, 64, 1, 1, 20))
    enc = wh.HIPEncoder(tensors, meta)
    ref = orc.OracleEncoder(tensors, meta)
    full = wh.synth.mel_input("efr", 16, T=41)
    got = enc.encode(full)
    assert got.shape == (20, 64)
    assert _rel(got, ref.encode(full)) < TOL
    assert _rel(got, enc.encode(full.reshape(-1)[:16 * 40].reshape(16, 40))) == 0.0
    with pytest.raises(wh.native.WhError, match=r"T=42 > 2\*n_audio_ctx=40"):
        enc.encode(np.zeros((16, 42), np.float32))
    with pytest.raises(wh.native.WhError, match="mel must be"):
        enc.encode(np.zeros((15, 8), np.float32))
    enc.close()


def test_encode_device_matches_host(wh, gpu):
    """wh_encode_device (mel and output in device memory) gives the bits of
    wh_encode: a full window, then a shorter one on the same handle (the
    workspace is reused), then the 2 n_ctx + 1 frame rule read in place."""
    dims = (16, 128, 2, 2, 40)
    tensors, meta = wh.synth.make_encoder("edev", 8, dims=dims)
    enc = wh.HIPEncoder(tensors, meta)
    out = wh.native.DevBuf(40 * 128 * 4)
    for T in (80, 37, 81):
        print(f"encode_device T={T}", flush=True)
        mel = wh.synth.mel_input("edev", 16, T=T)
        want = enc.encode(mel)
        dmel = wh.native.DevBuf.from_array(mel)
        rows = enc.encode_device(dmel.ptr.value, 16, T, out.ptr.value, 40)
        assert rows == want.shape[0] == min((T + 1) // 2, 40)
        got = out.download((40, 128), np.float32)[:rows]
        assert np.array_equal(got, want), T
        dmel.free()
    with pytest.raises(wh.native.WhError, match="output capacity"):
        enc.encode_device(out.ptr.value, 16, 80, out.ptr.value, 39)
    out.free()
    enc.close()


def test_encoder_cancelled(wh, gpu):
    """encoder_test.go:95-110: a cancelled context stops Encode with a
    cancellation error."""
    tensors, meta = wh.synth.make_encoder("ecan", 8, dims=(16, 64, 1, 2, 20))
    enc = wh.HIPEncoder(tensors, meta)
    flag = C.c_int32(1)
    with pytest.raises(wh.CancelledError, match="context canceled"):
        enc.encode(wh.synth.mel_input("ecan", 16, T=40), cancel=flag)
    flag.value = 0
    assert enc.encode(wh.synth.mel_input("ecan", 16, T=40), cancel=flag).shape == (20, 64)
    enc.close()


def _enc_meta_kv(meta):
    keys = {"n_head": "whisper.encoder.attention.head_count", "n_layer": "whisper.encoder.layer_count",
            "n_ctx": "whisper.encoder.context_length", "n_state": "whisper.encoder.embedding_length",
            "n_mels": "whisper.audio.mel_count"}
    return [(keys[k], 4, int(v)) for k, v in meta.items()]


@pytest.mark.parametrize("with_meta", [True, False])
def test_encoder_from_gguf(wh, gpu, tmp_path, with_meta):
    """The encoder and decoder tensors of one GGUF file: wh_encoder_load_gguf
    reads the encoder's (with whisper.encoder.* metadata or inferring it) and
    encodes like the tensor-table handle."""
    dims = (16, 128, 2, 2, 50)
    et, em = wh.synth.make_encoder("egg", 8, dims=dims)
    dt, dm = wh.synth.make_decoder("egg", 8, dims=(400, 128, 2, 1, 32))
    mel = wh.synth.mel_input("egg", 16, T=100)
    base = wh.HIPEncoder(et, em)
    want = base.encode(mel)
    base.close()
    path = str(tmp_path / "model.gguf")
    wh.synth.write_gguf(path, et + dt, dm if with_meta else None, extra=_enc_meta_kv(em) if with_meta else None)
    enc = wh.HIPEncoder.from_gguf(path)
    assert (enc.n_mels, enc.n_state, enc.n_head, enc.n_layer, enc.n_ctx) == dims
    assert np.array_equal(enc.encode(mel), want)
    enc.close()
    dec = wh.HIPDecoder.from_gguf(path)
    assert dec.n_state == 128
    dec.close()


def test_tiny_en_full_size_vs_oracle(wh, orc, gpu):
    """tiny.en (80 mels, d = 384, 6 heads, 4 layers) on a full 30 s window of
    3000 frames -> 1500 encoder rows, against the oracle."""
    tensors, meta = wh.synth.make_encoder("tiny.en", 8)
    mel = wh.synth.mel_input("tiny.en", 80, T=3000)
    enc = wh.HIPEncoder(tensors, meta)
    got = enc.encode(mel)
    enc.close()
    want = orc.OracleEncoder(tensors, meta, threads=16).encode(mel)
    assert got.shape == want.shape == (1500, 384)
    print(f"tiny.en encoder rel err {_rel(got, want):.3g}", flush=True)
    assert _rel(got, want) < TOL


def test_large_v3_shape_vs_oracle(wh, orc, gpu):
    """The large-v3 encoder's shapes (128 mels, d = 1280, 20 heads) over a full
    window of 3000 frames -> 1500 rows, with its first block only (every block
    runs the same kernels at the same sizes), Q8_0, against the oracle."""
    dims = (128, 1280, 20, 1, 1500)
    tensors, meta = wh.synth.make_encoder("large-v3", 8, dims=dims)
    mel = wh.synth.mel_input("large-v3", 128, T=3000)
    enc = wh.HIPEncoder(tensors, meta)
    got = enc.encode(mel)
    enc.close()
    want = orc.OracleEncoder(tensors, meta, threads=16).encode(mel)
    assert got.shape == want.shape == (1500, 1280)
    print(f"large-v3 shape encoder rel err {_rel(got, want):.3g}", flush=True)
    assert _rel(got, want) < TOL


def test_device_encoder_output_feeds_decoder(wh, gpu):
    """mel -> wh_encode_device -> wh_decode_device, the encoder output never
    leaving HBM, gives the tokens of the host-buffer path (greedy and beam 3);
    a host pointer is rejected."""
    dims_e, dims_d = (16, 128, 2, 2, 60), (600, 128, 2, 2, 48)
    et, em = wh.synth.make_encoder("edd", 8, dims=dims_e)
    dt, dm = wh.synth.make_decoder("edd", 8, dims=dims_d)
    mel = wh.synth.mel_input("edd", 16, T=120)
    enc, dec = wh.HIPEncoder(et, em), wh.HIPDecoder(dt, dm)
    host = enc.encode(mel)
    dmel = wh.native.DevBuf.from_array(mel)
    dout = wh.native.DevBuf(60 * 128 * 4)
    rows = enc.encode_device(dmel.ptr.value, 16, 120, dout.ptr.value, 60)
    assert rows == 60
    for beam in (1, 3):
        p = wh.DecoderParams(prompt=[5, 6, 7], beam_size=beam, max_tokens=16, no_fallback=True)
        assert dec.decode_tokens_device(dout.ptr.value, rows, p) == dec.decode_tokens(host, p), beam
    with pytest.raises(wh.native.WhError, match="not device memory"):
        dec.decode_tokens_device(host.ctypes.data, rows, wh.DecoderParams(prompt=[5, 6, 7], max_tokens=4))
    dmel.free()
    dout.free()
    enc.close()
    dec.close()


def test_mel_to_tokens_end_to_end(wh, orc, gpu):
    """mel -> device encoder -> device decoder gives the tokens of mel -> oracle
    encoder -> oracle decoder (greedy and beam 3)."""
    dims_e, dims_d = (16, 128, 2, 2, 60), (600, 128, 2, 2, 48)
    et, em = wh.synth.make_encoder("e2e", 8, dims=dims_e)
    dt, dm = wh.synth.make_decoder("e2e", 8, dims=dims_d)
    mel = wh.synth.mel_input("e2e", 16, T=120)
    enc, dec = wh.HIPEncoder(et, em), wh.HIPDecoder(dt, dm)
    e_dev = enc.encode(mel)
    e_ref = orc.OracleEncoder(et, em).encode(mel)
    ref = orc.OracleModel(dt, dm)
    for beam in (1, 3):
        p = wh.DecoderParams(prompt=[5, 6, 7], beam_size=beam, max_tokens=16, no_fallback=True)
        assert dec.decode_tokens(e_dev, p) == ref.decode(e_ref, p), beam
    enc.close()
    dec.close()
