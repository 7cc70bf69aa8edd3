"""The oracle encoder (internal/model/encoder.go:265-396, ml/conv.go:19-70)
pinned against the reference's Conv1D known answer, closed forms of the
convolution's padding and stride, the reference's encoder test behaviours
(output length, T = 2 n_ctx + 1 truncation, T > 2 n_ctx rejected) and an
independent float64 numpy restatement of the whole encoder."""
import math

import numpy as np
import pytest


def _deq(orc, t):
    n = int(np.prod(t.shape))
    return orc.dequantize(t.data, t.type, n).astype(np.float64).reshape(t.shape)


def _ln(x, w, b):
    m = x.mean(axis=-1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=-1, keepdims=True)
    return (x - m) / np.sqrt(v + 1e-5) * w + b


def _gelu(x):
    return 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def _conv(x, w, b, stride):
    """Zero-padded 1-D convolution, kernel 3, padding 1, as a sum of shifted products."""
    cin, T = x.shape
    xp = np.concatenate([np.zeros((cin, 1)), x, np.zeros((cin, 1))], axis=1)
    tp = (T + 2 - 3) // stride + 1
    out = np.empty((w.shape[0], tp))
    for t in range(tp):
        win = xp[:, t * stride:t * stride + 3]  # [cin, 3]
        out[:, t] = np.tensordot(w, win, axes=([1, 2], [0, 1])) + b
    return out


def numpy_encoder(W, meta, mel):
    """encoder.go:265-396 in float64, exact softmax."""
    d, H, L = meta["n_state"], meta["n_head"], meta["n_layer"]
    hd = d // H
    x = _gelu(_conv(mel.astype(np.float64), W["encoder.conv1.weight"], W["encoder.conv1.bias"], 1))
    x = _gelu(_conv(x, W["encoder.conv2.weight"], W["encoder.conv2.bias"], 2)).T
    T = x.shape[0]
    x = x + W["encoder.positional_embedding"][:T]
    for i in range(L):
        p = f"encoder.blocks.{i}."
        h = _ln(x, W[p + "attn_ln.weight"], W[p + "attn_ln.bias"])
        q = h @ W[p + "attn.query.weight"].T + W[p + "attn.query.bias"]
        k = h @ W[p + "attn.key.weight"].T
        v = h @ W[p + "attn.value.weight"].T + W[p + "attn.value.bias"]
        att = np.empty_like(q)
        for j in range(H):
            sl = slice(j * hd, (j + 1) * hd)
            s = q[:, sl] @ k[:, sl].T / math.sqrt(hd)
            s = np.exp(s - s.max(axis=1, keepdims=True))
            att[:, sl] = (s / s.sum(axis=1, keepdims=True)) @ v[:, sl]
        x = x + att @ W[p + "attn.out.weight"].T + W[p + "attn.out.bias"]
        h = _ln(x, W[p + "mlp_ln.weight"], W[p + "mlp_ln.bias"])
        h = _gelu(h @ W[p + "mlp.0.weight"].T + W[p + "mlp.0.bias"])
        x = x + h @ W[p + "mlp.2.weight"].T + W[p + "mlp.2.bias"]
    return _ln(x, W["encoder.ln_post.weight"], W["encoder.ln_post.bias"])


def test_conv1d_reference_known_answer(orc):
    """ml/ops_test.go:316-347: the [1, 0, -1] edge detector over 1..5."""
    got = orc.conv1d(np.array([[1, 2, 3, 4, 5]], np.float32), np.array([[[1, 0, -1]]], np.float32),
                     np.zeros(1, np.float32), 1)
    assert got.tolist() == [[-2, -2, -2, -2, 4]]


def test_conv1d_padding_and_stride(orc):
    """Delta kernels pick shifted inputs: [0,1,0] at stride 2 gives x[2t], [1,0,0]
    gives x[2t-1] with a zero at t = 0, [0,0,1] gives x[2t+1] (zero past the end);
    T' = (T - 1) // 2 + 1 for odd and even T."""
    for T in (7, 8):
        x = np.arange(1, T + 1, dtype=np.float32)[None]
        for kern, want in (([0, 1, 0], x[0, 0::2]), ([1, 0, 0], np.r_[0, x[0, 1::2]][:(T - 1) // 2 + 1]),
                           ([0, 0, 1], np.r_[x[0, 1::2], 0][:(T - 1) // 2 + 1])):
            got = orc.conv1d(x, np.array([[kern]], np.float32), np.zeros(1, np.float32), 2)
            assert got.shape == (1, (T - 1) // 2 + 1)
            assert got[0].tolist() == list(want), (T, kern)
    # channels and bias: out[o, t] = b[o] + sum_c w[o, c, 1] x[c, t] for a centre-only kernel
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 6)).astype(np.float32)
    w = np.zeros((2, 3, 3), np.float32)
    w[:, :, 1] = rng.standard_normal((2, 3))
    b = np.array([0.5, -1.0], np.float32)
    got = orc.conv1d(x, w, b, 1)
    assert np.allclose(got, w[:, :, 1] @ x + b[:, None], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("qtype", [8, 3, 0])
def test_encoder_matches_numpy_restatement(wh, orc, qtype):
    dims = (16, 128, 2, 2, 60)
    tensors, meta = wh.synth.make_encoder(f"enp{qtype}", qtype, dims=dims)
    mel = wh.synth.mel_input(f"enp{qtype}", 16, T=120)
    ref = orc.OracleEncoder(tensors, meta)
    ref.set_fast_exp(False)
    got = ref.encode(mel)
    W = {t.name: _deq(orc, t) for t in tensors}
    want = numpy_encoder(W, meta, mel)
    assert got.shape == want.shape == (60, 128)
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 2e-5, qtype


def test_encoder_fast_exp_is_the_default(wh, orc):
    """The encoder's attention softmax takes the fast exp by default
    (attention.go:14): the output differs from the exact-exp one by more than
    rounding and far less than the values."""
    tensors, meta = wh.synth.make_encoder("efx", 8, dims=(16, 128, 2, 1, 40))
    mel = wh.synth.mel_input("efx", 16, T=80)
    ref = orc.OracleEncoder(tensors, meta)
    a = ref.encode(mel)
    ref.set_fast_exp(False)
    b = ref.encode(mel)
    diff = np.max(np.abs(a - b)) / np.max(np.abs(b))
    assert 1e-8 < diff < 1e-3


def test_encoder_lengths_and_limits(wh, orc):
    """encoder.go:268-282 and encoder_test.go:79-93: T frames give T/2 output
    rows (odd T: (T + 1) / 2); T = 2 n_ctx + 1 keeps the first n_mels * 2 n_ctx
    values of the row-major buffer (the reference re-slices the flat data, so
    band b then starts b values early); T > 2 n_ctx is an error; a mel with the
    wrong band count is an error."""
    tensors, meta = wh.synth.make_encoder("elen", 8, dims=(16, 64, 1, 1, 20))
    ref = orc.OracleEncoder(tensors, meta)
    full = wh.synth.mel_input("elen", 16, T=41)
    assert ref.encode(full[:, :8]).shape == (4, 64)
    assert ref.encode(full[:, :7]).shape == (4, 64)
    assert np.array_equal(ref.encode(full), ref.encode(full.reshape(-1)[:16 * 40].reshape(16, 40)))
    assert not np.array_equal(ref.encode(full), ref.encode(full[:, :40]))
    with pytest.raises(RuntimeError, match=r"T=42 > 2\*n_audio_ctx=40"):
        ref.encode(np.zeros((16, 42), np.float32))
    with pytest.raises(RuntimeError, match="mel must be"):
        ref.encode(np.zeros((15, 8), np.float32))


def test_encoder_hparams_inferred_and_layouts(wh, orc):
    """encoder.go:63-170: without metadata the sizes come from the tensors
    (head count d / 64); the legacy [n_mels, d, 3] conv1 order and a [d, n_ctx]
    positional embedding load to the same encoder."""
    tensors, meta = wh.synth.make_encoder("einf", 0, dims=(16, 128, 2, 1, 30))
    mel = wh.synth.mel_input("einf", 16, T=60)
    want = orc.OracleEncoder(tensors, meta).encode(mel)
    e = orc.OracleEncoder(tensors, None)
    assert (e.n_mels, e.n_state, e.n_head, e.n_layer, e.n_ctx) == (16, 128, 2, 1, 30)
    alt = []
    for t in tensors:
        x = t.data.view(np.float32).reshape(t.shape)
        if t.name == "encoder.conv1.weight":
            alt.append(wh.synth.Tensor(t.name, 0, (16, 128, 3), np.ascontiguousarray(x.transpose(1, 0, 2))))
        elif t.name == "encoder.positional_embedding":
            alt.append(wh.synth.Tensor(t.name, 0, (128, 30), np.ascontiguousarray(x.T)))
        else:
            alt.append(t)
    got = orc.OracleEncoder(alt, meta).encode(mel)
    assert np.array_equal(got, want)
