"""HIP path vs the CPU oracle, through the C ABI (libwhisper_hip.so).

Bars: bit-exact dequantisation; logits within 1e-3 of the oracle measured as
max|gpu - oracle| / max|oracle| (fp32 accumulation on both sides); identical
token sequences for greedy, beam and batched decoding.
"""
import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

QTYPES = [8, 2, 3, 6, 7]
LOGIT_TOL = 1e-3


def _special_f16_blocks(qtype, nblk, rng):
    """Random raw blocks whose scale words include zero, subnormal, max and
    negative f16 values (NaN/Inf excluded from products)."""
    bb = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}[qtype]
    raw = rng.integers(0, 256, size=nblk * bb, dtype=np.uint8)
    specials = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x1234, 0x8001]
    for b in range(nblk):
        h = specials[b % len(specials)] if b < 3 * len(specials) else int(rng.integers(0, 0x7C00))
        raw[b * bb] = h & 0xFF
        raw[b * bb + 1] = h >> 8
        if qtype in (3, 7):
            m = specials[(b + 3) % len(specials)]
            raw[b * bb + 2] = m & 0xFF
            raw[b * bb + 3] = m >> 8
    return raw


@pytest.mark.parametrize("qtype", QTYPES + [1, 0])
def test_dequant_bit_exact(wh, orc, gpu, qtype):
    rng = np.random.default_rng(qtype)
    for n in (32, 1000, 4096 + 7):
        if qtype in (0, 1):
            raw = rng.integers(0, 256, size=n * (4 if qtype == 0 else 2), dtype=np.uint8)
            if qtype == 0:  # avoid NaN patterns (NaN != NaN for the comparison)
                raw = np.frombuffer(rng.standard_normal(n).astype(np.float32).tobytes(), np.uint8).copy()
        else:
            raw = _special_f16_blocks(qtype, (n + 31) // 32, rng)
        got = wh.quant.dequantize_device(qtype, raw, n)
        want = orc.dequantize(raw, qtype, n)
        assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist(), f"type {qtype} n {n}"


def test_dequant_reference_kats(wh, gpu):
    """The one-block KATs of internal/gguf/gguf_test.go:190-309 on the device."""
    import json, os
    kats = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "dequant_kats.json")))
    for k in kats:
        raw = np.array(k["block"], np.uint8)
        got = wh.quant.dequantize_device(k["type"], raw, 32)
        for i, v in k["expect"].items():
            assert got[int(i)] == np.float32(v), (k["name"], i)


@pytest.mark.parametrize("qtype", QTYPES + [0])
@pytest.mark.parametrize("shape", [(64, 128), (1280, 1280), (96, 5120), (37, 100), (300, 384), (20, 50)])
@pytest.mark.parametrize("batch", [1, 2, 3, 5, 7, 16])
def test_gemv_vs_oracle(wh, orc, gpu, qtype, shape, batch):
    """Batch 1, 2 and 3..5 (the last two staged with zero rows) take the LDS-staged
    kernels on matrices of >= 1024 rows and the register-sliced one below; 7 and 16
    the matrix-core kernel (7 with zero rows); (96, 5120) stages x in column chunks;
    (20, 50) has rows of x that are not 16-byte aligned."""
    rows, cols = shape
    rng = np.random.default_rng(rows * 7 + cols + qtype)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    raw = wh.quant.quantize_rows(qtype, w) if qtype else w.reshape(-1).view(np.uint8)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    mat = wh.native.lib()
    import ctypes as C
    h = C.c_void_p()
    wh.native.check(mat.wh_matrix_create(qtype, rows, cols, raw.ctypes.data, raw.size, 0, C.byref(h)))
    try:
        xb = wh.native.DevBuf.from_array(x)
        yb = wh.native.DevBuf(batch * rows * 4)
        wh.native.check(mat.wh_gemv(h, xb.ptr, batch, yb.ptr, None))
        got = yb.download((batch, rows), np.float32)
    finally:
        mat.wh_matrix_destroy(h)
    want = orc.gemv(qtype, raw, rows, cols, x)
    # float64 brute force of the same dequantised weights bounds both
    rb = orc.row_bytes(qtype, cols)
    deq = np.stack([orc.dequantize(raw[r * rb:(r + 1) * rb], qtype, cols) for r in range(rows)]).astype(np.float64)
    exact = x.astype(np.float64) @ deq.T
    scale = np.max(np.abs(exact)) + 1e-30
    assert np.max(np.abs(got - exact)) / scale < 2e-5
    assert np.max(np.abs(want - exact)) / scale < 2e-5


def _model(wh, name, qtype, dims):
    tensors, meta = wh.synth.make_decoder(name, qtype, dims=dims)
    return tensors, meta


MODEL_CASES = [
    ("m64q8", 8, (2048, 128, 2, 2, 64), 96),     # hd 64, chunked cross-attention
    ("m64q41", 3, (1500, 192, 3, 2, 48), 150),   # Q4_1
    ("m64q51", 7, (1000, 128, 2, 1, 40), 60),    # Q5_1
    ("m64q40", 2, (1000, 128, 2, 1, 40), 256),   # Q4_0, several key chunks
    ("m64q50", 6, (1000, 128, 2, 1, 40), 130),   # Q5_0, ragged last chunk
    ("hd32", 8, (777, 96, 3, 2, 32), 30),        # head size 32: generic attention
    ("f32", 0, (500, 64, 2, 1, 32), 20),         # float weights
    ("ragT64", 8, (900, 192, 3, 1, 40), 100),    # 3 heads over 100 frames: head slabs start inside rows
    ("ragT32", 8, (777, 96, 3, 1, 32), 31),      # the same with head size 32
]


@pytest.mark.parametrize("name,qtype,dims,enc_len", MODEL_CASES)
def test_forward_logits_vs_oracle(wh, orc, gpu, name, qtype, dims, enc_len):
    tensors, meta = _model(wh, name, qtype, dims)
    d = dims[1]
    enc = wh.synth.encoder_output(name, d, enc_len=enc_len)
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    for prompt in ([7], [3, 9, 11]):
        seq = dec.sequence([enc])
        seq.set_tokens(0, prompt)
        st = ref.state(prompt)
        for step in range(4):
            ids, logits = seq.step_greedy(logits=True)
            want = st.forward(enc)
            assert rel_err(logits[0], want) < LOGIT_TOL, (name, prompt, step)
            st.push(ids[0])
            prompt = prompt + [ids[0]]
        seq.close()
    dec.close()


@pytest.mark.parametrize("name,qtype,dims,enc_len", MODEL_CASES[:4])
def test_greedy_tokens_identical(wh, orc, gpu, name, qtype, dims, enc_len):
    tensors, meta = _model(wh, name, qtype, dims)
    enc = wh.synth.encoder_output(name, dims[1], enc_len=enc_len)
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    for prompt in ([1], [50 % dims[0], 2, 3]):
        p = wh.DecoderParams(prompt=prompt, max_tokens=24, no_fallback=True)
        assert dec.decode_tokens(enc, p) == ref.decode(enc, p)


def test_beam_tokens_identical(wh, orc, gpu):
    tensors, meta = _model(wh, "beam", 7, (1200, 128, 2, 2, 48))
    enc = wh.synth.encoder_output("beam", 128, enc_len=100)
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    p = wh.DecoderParams(prompt=[5, 6, 7], beam_size=5, max_tokens=16, no_fallback=True)
    assert dec.decode_tokens(enc, p) == ref.decode(enc, p)


def test_beam_tied_logits(wh, orc, gpu):
    """Token-embedding rows repeated with period 7 give every logit value ~170
    times (the logits matrix is the embedding), so every step's top-k holds
    equal values: the kept tokens and their order are those of the reference's
    replace-min scan (decoder.go:1089-1127), which the device reruns for such
    rows, not the (value, index) order of the plain top-k."""
    tensors, meta = _model(wh, "beamtie", 7, (1200, 128, 2, 2, 48))
    for t in tensors:
        if t.name == "decoder.token_embedding.weight":
            rows = t.data.reshape(t.shape[0], -1)
            rows[:] = rows[np.arange(t.shape[0]) % 7]
    enc = wh.synth.encoder_output("beamtie", 128, enc_len=100)
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    p = wh.DecoderParams(prompt=[5, 6, 7], beam_size=5, max_tokens=12, no_fallback=True)
    got = dec.decode_tokens(enc, p)
    assert got == ref.decode(enc, p)
    assert len(got) > 3


def test_batch_of_seven_streams(wh, orc, gpu):
    """Seven streams (the matrix-core GEMV at batch 7, ragged prompts) against the
    oracle's single-stream decode of each."""
    tensors, meta = _model(wh, "batch7", 7, (1200, 128, 2, 2, 64))
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    encs = [wh.synth.encoder_output("batch7", 128, stream=i, enc_len=60) for i in range(7)]
    params = [wh.DecoderParams(prompt=list(range(3, 4 + 2 * i)), max_tokens=10, no_fallback=True) for i in range(7)]
    got = dec.decode_batch(encs, params)
    for i in range(7):
        assert got[i] == ref.decode(encs[i], params[i]), i


def test_batch_equals_single_streams(wh, orc, gpu):
    tensors, meta = _model(wh, "batch", 3, (1000, 128, 2, 2, 64))
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    encs = [wh.synth.encoder_output("batch", 128, stream=i, enc_len=80) for i in range(4)]
    params = [wh.DecoderParams(prompt=list(range(1, 2 + 3 * i)), max_tokens=12, no_fallback=True) for i in range(4)]
    got = dec.decode_batch(encs, params)
    for i in range(4):
        assert got[i] == ref.decode(encs[i], params[i]), i


@pytest.mark.parametrize("qtype,dims", [(3, (1000, 512, 8, 2, 64)), (8, (1000, 512, 8, 2, 64)),
                                        (2, (1000, 512, 8, 2, 64)), (6, (1000, 512, 8, 2, 64)),
                                        (7, (1000, 512, 8, 2, 64)), (3, (1000, 768, 12, 1, 64))])
def test_sixteen_streams_split_gemv_vs_oracle(wh, orc, gpu, qtype, dims):
    """16 streams on the multi-kernel chain: the matrix-core GEMV at batch 16 with
    K split over several workgroups per 16-row tile (d = 512: 2 ranges of the
    512-column rows, 4 of the 2048-column fc2 rows; d = 768: fc1's 3072 rows take
    the taller matrices' kernel, 3 ranges), the last workgroup of a tile summing
    the partial tiles; every stream's logits at every step against the oracle."""
    d = dims[1]
    name = f"s16split{qtype}_{d}"
    tensors, meta = _model(wh, name, qtype, dims)
    encs = [wh.synth.encoder_output(name, d, stream=i, enc_len=48) for i in range(16)]
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    seq = dec.sequence(encs)
    prompts = [[3 + i, 7, 11 + 2 * i][:1 + i % 3] for i in range(16)]
    for i, p in enumerate(prompts):
        seq.set_tokens(i, p)
    states = [ref.state(p) for p in prompts]
    for step in range(4):
        ids, lg = seq.step_greedy(logits=True)
        for i in range(16):
            want = states[i].forward(encs[i])
            assert rel_err(lg[i], want) < LOGIT_TOL, (step, i, rel_err(lg[i], want))
            states[i].push(ids[i])
    seq.close()
    dec.close()


def test_reference_test_fixture(wh, orc, gpu):
    """internal/model/decoder_test.go:89-180 on the device: d=4, 2 heads of 2,
    8 encoder frames, V=51865; greedy and beam return non-empty segments and
    match the oracle token for token."""
    tensors, meta = wh.synth.reference_test_decoder()
    enc = np.full((8, 4), 0.01, np.float32)
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    p = wh.DecoderParams(prompt=[50258, 50259, 50357, 50363], beam_size=1, max_tokens=5, temperature=1.0)
    segs = dec.decode(enc, p)
    assert len(segs) == 1 and len(segs[0].tokens) > 0
    assert dec.decode_tokens(enc, p) == ref.decode(enc, p)
    p.beam_size = 3
    assert dec.decode_tokens(enc, p) == ref.decode(enc, p)


@pytest.mark.parametrize("dims,steps", [
    ((800, 128, 2, 1, 96), 70),   # head size 64: LDS-tiled kernel, past one 64-key tile
    ((600, 96, 3, 2, 80), 66),    # head size 32, two layers
    ((500, 320, 2, 1, 40), 20),   # head size 160: the one-wave kernel
])
def test_textbook_attention_mode_vs_numpy(wh, orc, gpu, dims, steps):
    """Opt-in mode 1 (textbook causal mask over the KV cache) against the float64
    numpy restatement of the same forward with the oracle's fast-exp softmax,
    at every greedy step from position 0. The restatement is pinned on the CPU
    against a whole-block forward through the oracle's causal SDPA. At position 0
    both modes see one key, so the first step equals the reference mode exactly;
    from position 1 the reference mode is far from the textbook logits."""
    from test_oracle_decoder import NumpyDecoder

    name = "mode1_%d_%d" % dims[1:3]
    tensors, meta = _model(wh, name, 8, dims)
    d = dims[1]
    enc = wh.synth.encoder_output(name, d, enc_len=40)
    dec = wh.HIPDecoder(tensors, meta)
    dec.set_attention_mode(1)
    seq = dec.sequence([enc])
    seq.set_tokens(0, [1])
    npd = NumpyDecoder(orc, tensors, meta, causal=True, fast=True)
    ref = NumpyDecoder(orc, tensors, meta, fast=True)
    toks = [1]
    for step in range(steps):
        ids, lg = seq.step_greedy(logits=True)
        want = npd.forward(toks, enc)
        ref_mode = ref.forward(toks, enc)
        assert rel_err(lg[0], want) < 1e-4, (step, rel_err(lg[0], want))
        if step > 0:
            assert rel_err(ref_mode, want) > 1e-2, step
        toks.append(int(ids[0]))
    # at position 0 both modes see one key: logits equal the reference mode
    dec2 = wh.HIPDecoder(tensors, meta)
    s2 = dec2.sequence([enc])
    s2.set_tokens(0, [1])
    _, m0 = s2.step_greedy(logits=True)
    s1 = dec.sequence([enc])
    s1.set_tokens(0, [1])
    _, l0 = s1.step_greedy(logits=True)
    assert rel_err(l0[0], m0[0]) < 1e-6


@pytest.mark.parametrize("temperature", [1.0, 0.7])
def test_step_topk_vs_oracle(wh, orc, gpu, temperature):
    """Per-row top-k and log-probabilities (decoder.go:1068-1136) on the device
    against the oracle's top-k of the same raw logits after the oracle's
    repetition penalty: a 51864-entry vocabulary, split over 26 partitions on the
    device, two streams with different histories."""
    tensors, meta = _model(wh, "topk", 8, (51864, 64, 2, 1, 32))
    encs = [wh.synth.encoder_output("topk", 64, stream=i, enc_len=40) for i in range(2)]
    dec = wh.HIPDecoder(tensors, meta)
    seq = dec.sequence(encs)
    prompts = [[50258, 50259, 50359], [11, 11, 503, 4096, 11]]
    for i, p in enumerate(prompts):
        seq.set_tokens(i, p)
    k = 6
    tok, lp, logits = seq.step_topk(k=k, temperature=temperature, logits=True)
    for i, p in enumerate(prompts):
        pen = orc.repetition_penalty(logits[i], np.array(p, np.int32))
        want_tok, want_lp = orc.topk(pen, k, temperature)
        assert tok[i].tolist() == want_tok.tolist(), i
        logz = float(np.log(np.sum(np.exp((pen / temperature).astype(np.float64) - np.max(pen / temperature))))) \
            + float(np.max(pen / temperature))
        assert np.max(np.abs(lp[i] - want_lp)) < 1e-5 * max(1.0, abs(logz)), (lp[i], want_lp)
    seq.close()
    dec.close()
