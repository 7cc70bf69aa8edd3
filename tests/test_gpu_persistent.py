"""Persistent decode kernel (whole greedy token steps in one cooperative launch)
against the multi-kernel path and the CPU oracle, through the C ABI.

Bars as for the multi-kernel path: logits within 1e-3 of the oracle
(max|gpu - oracle| / max|oracle|) and identical token sequences, including the
reference's stop rules (decoder.go:441-485). Every test first checks that the
persistent kernel really served the sequence (launch counter), so a silent
multi-kernel fallback fails the test.
"""
import contextlib
import os

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3

# (name, type, (n_vocab, n_state, n_head, n_layer, n_ctx), encoder frames)
CASES = [
    ("pq8", 8, (2048, 128, 2, 2, 64), 96),       # one key chunk
    ("pq40", 2, (1000, 128, 2, 1, 64), 300),     # two chunks, ragged
    ("pq41", 3, (1500, 192, 3, 2, 64), 150),
    ("pq50", 6, (1000, 256, 4, 2, 64), 513),     # three chunks, one row in the last
    ("pq51", 7, (1200, 128, 2, 2, 64), 1500),    # six chunks of 250 frames
]


@contextlib.contextmanager
def persistent(on):
    """The path is chosen when a sequence is created (WHISPER_HIP_PERSISTENT)."""
    old = os.environ.get("WHISPER_HIP_PERSISTENT")
    os.environ["WHISPER_HIP_PERSISTENT"] = "1" if on else "0"
    try:
        yield
    finally:
        if old is None:
            del os.environ["WHISPER_HIP_PERSISTENT"]
        else:
            os.environ["WHISPER_HIP_PERSISTENT"] = old


def _setup(wh, name, qtype, dims, enc_len):
    tensors, meta = wh.synth.make_decoder(name, qtype, dims=dims)
    enc = wh.synth.encoder_output(name, dims[1], enc_len=enc_len)
    return tensors, meta, enc


@pytest.mark.parametrize("name,qtype,dims,enc_len", CASES)
def test_persistent_logits_vs_oracle(wh, orc, gpu, name, qtype, dims, enc_len):
    tensors, meta, enc = _setup(wh, name, qtype, dims, enc_len)
    print(f"case {name} type {qtype} dims {dims} enc {enc_len}", flush=True)
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    prompt = [3, 9, 11]
    with persistent(True):
        seq = dec.sequence([enc])
    assert seq.persistent[0]
    seq.set_tokens(0, prompt)
    st = ref.state(prompt)
    for step in range(5):
        ids, logits = seq.step_greedy(logits=True)
        want = st.forward(enc)
        assert rel_err(logits[0], want) < LOGIT_TOL, (name, step)
        cur = orc.repetition_penalty(want, np.array(prompt, np.int32))
        assert ids[0] == int(orc.sample_greedy(cur, 1.0, eot=50256)), (name, step)
        st.push(ids[0])
        prompt = prompt + [ids[0]]
    assert seq.persistent[1] == 5
    seq.close()
    dec.close()


@pytest.mark.parametrize("name,qtype,dims,enc_len", CASES)
def test_persistent_generate_matches_multikernel_and_oracle(wh, orc, gpu, name, qtype, dims, enc_len):
    """Many steps in one launch == one multi-kernel step per token == oracle."""
    tensors, meta, enc = _setup(wh, name, qtype, dims, enc_len)
    print(f"case {name}", flush=True)
    dec = wh.HIPDecoder(tensors, meta)
    prompt = [5, 6, 7]
    n = dims[4] - len(prompt) - 2
    with persistent(False):
        s0 = dec.sequence([enc])
    assert not s0.persistent[0]
    s0.set_tokens(0, prompt)
    want = s0.generate(n)
    s0.close()
    with persistent(True):
        s1 = dec.sequence([enc])
    s1.set_tokens(0, prompt)
    got = s1.generate(n)
    assert s1.persistent[1] >= 1
    s1.close()
    assert got == want
    ref = orc.OracleModel(tensors, meta)
    p = wh.DecoderParams(prompt=prompt, max_tokens=n, no_fallback=True)
    assert prompt + got == ref.decode(enc, p)[:len(prompt) + len(got)]
    dec.close()


def test_persistent_stop_rules(wh, gpu):
    """EOT stops the launch at the EOT token (decoder.go:462-470); max_len
    stops it when the history reaches that many tokens."""
    name, qtype, dims, enc_len = CASES[0]
    tensors, meta, enc = _setup(wh, name, qtype, dims, enc_len)
    dec = wh.HIPDecoder(tensors, meta)
    prompt = [1, 2]
    with persistent(False):
        s0 = dec.sequence([enc])
    s0.set_tokens(0, prompt)
    free = s0.generate(30)
    s0.close()
    assert len(free) == 30
    # make the 12th generated token the end-of-text id
    eot = free[11]
    first = free.index(eot)
    dec.set_vocabulary(eot)
    with persistent(True):
        s1 = dec.sequence([enc])
    s1.set_tokens(0, prompt)
    got = s1.generate(30)
    assert s1.persistent[1] >= 1
    assert got == free[:first + 1]
    s1.close()
    dec.set_vocabulary(50256)
    with persistent(True):
        s2 = dec.sequence([enc])
    s2.set_tokens(0, prompt)
    got = s2.generate(30, max_len=len(prompt) + 9)
    assert got == free[:9]
    s2.close()
    dec.close()


def test_persistent_decode_api(wh, orc, gpu):
    """Decode (the model.Decoder entry) on the persistent path equals the
    oracle's decode, and later decodes on the same model stay consistent."""
    name, qtype, dims, enc_len = CASES[2]
    tensors, meta, enc = _setup(wh, name, qtype, dims, enc_len)
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    for prompt in ([50 % dims[0], 2, 3], [9, 8]):
        p = wh.DecoderParams(prompt=prompt, max_tokens=40, no_fallback=True)
        with persistent(True):
            got = dec.decode_tokens(enc, p)
        assert got == ref.decode(enc, p)
    dec.close()


def test_persistent_large_v3_q8_0(wh, orc, gpu):
    """The benchmark workload (large-v3, Q8_0, 1500 frames): persistent and
    multi-kernel paths give the same 64 tokens; the first persistent step's
    logits match the oracle."""
    tensors, meta = wh.synth.make_decoder("large-v3", 8)
    enc = wh.synth.encoder_output("large-v3", meta["n_state"], stream=0)
    prompt = list(wh.synth.SOT_EN_TRANSCRIBE)
    dec = wh.HIPDecoder(tensors, meta)
    with persistent(False):
        s0 = dec.sequence([enc])
    s0.set_tokens(0, prompt)
    want = s0.generate(64)
    s0.close()
    with persistent(True):
        s1 = dec.sequence([enc])
    assert s1.persistent[0]
    s1.set_tokens(0, prompt)
    got = s1.generate(64)
    s1.close()
    assert got == want
    # logits of one persistent step against the oracle
    with persistent(True):
        s2 = dec.sequence([enc])
    s2.set_tokens(0, prompt + want[:2])
    _, logits = s2.step_greedy(logits=True)
    assert s2.persistent[1] == 1
    s2.close()
    ref = orc.OracleModel(tensors, meta, threads=16)
    st = ref.state(prompt + want[:2])
    assert rel_err(logits[0], st.forward(enc)) < LOGIT_TOL
    dec.close()
