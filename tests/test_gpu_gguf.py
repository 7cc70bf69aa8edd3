"""GGUF files through wh_model_load_gguf, end to end, and cancellation.

The reference builds its decoder from a GGUF file (whisper.go:138-181 ->
internal/gguf/gguf.go:52-135 -> internal/model/decoder.go:97-303). Three file
forms decode to the same tokens as the tensor-table model and the oracle:
canonical names with metadata; the HF alias names (internal/model/compat.go:
31-148); and no metadata at all, as cmd/quantize writes it
(cmd/quantize/main.go:65-119), so every hyper-parameter is inferred from tensor
shapes and the head count falls back to d/64 (decoder.go:107-164). Metadata of
other types than uint32 (strings, arrays, floats: what the reference's writer
may emit) is skipped by the parser.
"""
import ctypes as C

import pytest

pytestmark = pytest.mark.gpu

SUFFIX_HF = {
    "self_attn_ln.weight": "self_attn_layer_norm.weight", "self_attn_ln.bias": "self_attn_layer_norm.bias",
    "self_attn.query.weight": "self_attn.q_proj.weight", "self_attn.query.bias": "self_attn.q_proj.bias",
    "self_attn.key.weight": "self_attn.k_proj.weight", "self_attn.value.weight": "self_attn.v_proj.weight",
    "self_attn.value.bias": "self_attn.v_proj.bias", "self_attn.out.weight": "self_attn.out_proj.weight",
    "self_attn.out.bias": "self_attn.out_proj.bias", "cross_attn_ln.weight": "encoder_attn_layer_norm.weight",
    "cross_attn_ln.bias": "encoder_attn_layer_norm.bias", "cross_attn.query.weight": "encoder_attn.q_proj.weight",
    "cross_attn.query.bias": "encoder_attn.q_proj.bias", "cross_attn.key.weight": "encoder_attn.k_proj.weight",
    "cross_attn.value.weight": "encoder_attn.v_proj.weight", "cross_attn.value.bias": "encoder_attn.v_proj.bias",
    "cross_attn.out.weight": "encoder_attn.out_proj.weight", "cross_attn.out.bias": "encoder_attn.out_proj.bias",
    "mlp_ln.weight": "final_layer_norm.weight", "mlp_ln.bias": "final_layer_norm.bias",
    "mlp.0.weight": "fc1.weight", "mlp.0.bias": "fc1.bias", "mlp.2.weight": "fc2.weight", "mlp.2.bias": "fc2.bias",
}
TOP_HF = {"decoder.token_embedding.weight": "model.decoder.embed_tokens.weight",
          "decoder.positional_embedding": "model.decoder.embed_positions.weight",
          "decoder.ln.weight": "model.decoder.layer_norm.weight", "decoder.ln.bias": "model.decoder.layer_norm.bias"}


def hf_name(name):
    if name in TOP_HF:
        return TOP_HF[name]
    _, _, idx, rest = name.split(".", 3)
    return f"model.decoder.layers.{idx}.{SUFFIX_HF[rest]}"


def _renamed(wh, tensors, fn):
    return [wh.synth.Tensor(fn(t.name), t.type, t.shape, t.data) for t in tensors]


@pytest.mark.parametrize("qtype", [8, 7])
def test_gguf_forms_decode_like_tensor_table(wh, orc, gpu, tmp_path, qtype):
    # d = 128 with 2 heads: the head count inferred without metadata (d/64) is the same
    dims = (900, 128, 2, 2, 48)
    tensors, meta = wh.synth.make_decoder(f"gguf{qtype}", qtype, dims=dims)
    enc = wh.synth.encoder_output(f"gguf{qtype}", 128, enc_len=90)
    p = wh.DecoderParams(prompt=[5, 6, 7], max_tokens=20, no_fallback=True)
    pb = wh.DecoderParams(prompt=[5, 6, 7], beam_size=3, max_tokens=8, no_fallback=True)
    base = wh.HIPDecoder(tensors, meta)
    want, want_b = base.decode_tokens(enc, p), base.decode_tokens(enc, pb)
    base.close()
    ref = orc.OracleModel(tensors, meta)
    assert want == ref.decode(enc, p) and want_b == ref.decode(enc, pb)
    extra = [("general.architecture", 8, "whisper"), ("general.file_type", 4, qtype),
             ("tokenizer.ggml.tokens", 9, (8, ["", "", ""])), ("whisper.audio.sample_rate", 6, 16000.0),
             ("general.quantized", 7, 1), ("general.size", 10, 12345)]
    forms = {
        "canonical": (tensors, meta, None),
        "hf_aliases": (_renamed(wh, tensors, hf_name), meta, extra),
        "no_metadata": (tensors, None, None),
        "hf_no_metadata": (_renamed(wh, tensors, hf_name), None, extra),
    }
    for form, (ts, m, ex) in forms.items():
        print(f"gguf {qtype} {form}", flush=True)
        path = str(tmp_path / f"{form}.gguf")
        wh.synth.write_gguf(path, ts, m, extra=ex)
        dec = wh.HIPDecoder.from_gguf(path)
        assert (dec.n_vocab, dec.n_state, dec.n_head, dec.n_layer, dec.n_ctx) == dims, form
        assert dec.decode_tokens(enc, p) == want, form
        assert dec.decode_tokens(enc, pb) == want_b, form
        dec.close()


def test_gguf_head_count_inferred_from_width(wh, orc, gpu, tmp_path):
    """Without metadata a 4-head d=128 file decodes as 2 heads (d/64), exactly
    as the reference infers it; the oracle built with the same inference agrees."""
    tensors, meta = wh.synth.make_decoder("gguf4h", 8, dims=(700, 128, 4, 1, 32))
    enc = wh.synth.encoder_output("gguf4h", 128, enc_len=40)
    path = str(tmp_path / "m.gguf")
    wh.synth.write_gguf(path, tensors, None)
    dec = wh.HIPDecoder.from_gguf(path)
    assert dec.n_head == 2
    ref = orc.OracleModel(tensors, None)
    assert ref.n_head == 2
    p = wh.DecoderParams(prompt=[1, 2], max_tokens=10, no_fallback=True)
    assert dec.decode_tokens(enc, p) == ref.decode(enc, p)
    dec.close()


@pytest.mark.parametrize("beam", [1, 5])
def test_cancelled_before_decode(wh, gpu, beam):
    """decoder_test.go:124-152: a context cancelled before Decode returns an
    error wrapping context.Canceled; here WH_ERR_CANCELLED."""
    tensors, meta = wh.synth.reference_test_decoder()
    import numpy as np
    enc = np.full((8, 4), 0.01, np.float32)
    dec = wh.HIPDecoder(tensors, meta)
    flag = C.c_int32(1)
    p = wh.DecoderParams(prompt=[50258, 50259, 50357, 50363], beam_size=beam, max_tokens=10)
    with pytest.raises(wh.CancelledError, match="cancel"):
        dec.decode_tokens(enc, p, cancel=flag)
    flag.value = 0
    assert len(dec.decode_tokens(enc, p, cancel=flag)) > 4
    with pytest.raises(wh.CancelledError):
        dec.decode_batch([enc, enc], [wh.DecoderParams(prompt=[1, 2], max_tokens=4)] * 2, cancel=C.c_int32(1))
    dec.close()
