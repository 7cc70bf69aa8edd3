"""Beam search, per-stream sampling parameters and SuppressNST on the device,
against the CPU oracle through the C ABI.

The beam prune follows the reference's in-place reuse of beam objects and Go's
sort.Slice order (internal/model/decoder.go:575-718); the oracle restatement of
both is pinned in tests/test_oracle_beam.py. Every case prints its name first,
so a failing run names it.
"""
import contextlib
import os

import pytest

from conftest import rel_err
from models import forced_repeat_model

pytestmark = pytest.mark.gpu

BEAM_MODELS = [
    ("bq51", 7, (1200, 128, 2, 2, 48), 100),
    ("bq80", 8, (2000, 128, 2, 1, 64), 96),
    ("bq40", 2, (900, 192, 3, 1, 64), 150),
]


def _setup(wh, orc, name, qtype, dims, enc_len):
    tensors, meta = wh.synth.make_decoder(name, qtype, dims=dims)
    enc = wh.synth.encoder_output(name, dims[1], enc_len=enc_len)
    return wh.HIPDecoder(tensors, meta), orc.OracleModel(tensors, meta), enc


@pytest.mark.parametrize("name,qtype,dims,enc_len", BEAM_MODELS)
@pytest.mark.parametrize("prompt", [[5, 6, 7], [9], [1, 2]])
def test_beam5_vs_oracle(wh, orc, gpu, name, qtype, dims, enc_len, prompt):
    print(f"beam5 {name} prompt {prompt}", flush=True)
    dec, ref, enc = _setup(wh, orc, name, qtype, dims, enc_len)
    p = wh.DecoderParams(prompt=prompt, beam_size=5, max_tokens=16, no_fallback=True)
    got = dec.decode_tokens(enc, p)
    assert got == ref.decode(enc, p)
    dec.close()


@pytest.mark.parametrize("beam", [2, 3, 8, 16])
def test_beam_sizes_vs_oracle(wh, orc, gpu, beam):
    """From 8 hypotheses on, 40+ candidates reach pdqsort's partitioning; 16
    hypotheses give 80 candidates (Tukey ninther pivots, shifting partial
    insertion sort)."""
    print(f"beam {beam}", flush=True)
    dec, ref, enc = _setup(wh, orc, *BEAM_MODELS[0])
    p = wh.DecoderParams(prompt=[5, 6, 7], beam_size=beam, max_tokens=10, no_fallback=True)
    assert dec.decode_tokens(enc, p) == ref.decode(enc, p)
    dec.close()


def test_beam_over_16_rejected(wh, gpu):
    dec, _, enc = _setup(wh, __import__("oracle.oracle").oracle, *BEAM_MODELS[0])
    with pytest.raises(wh.native.WhError) as e:
        dec.decode_tokens(enc, wh.DecoderParams(prompt=[5], beam_size=17, max_tokens=2, no_fallback=True))
    assert e.value.code == wh.native.WH_ERR_UNSUPPORTED
    dec.close()


def test_beam_eot_carry_vs_oracle(wh, orc, gpu):
    """EOT set to a token the hypotheses reach after a few steps: finished
    hypotheses propose themselves with log-probability 0 and are carried over
    (decoder.go:581-590, :644-651) while the others continue."""
    dec, ref, enc = _setup(wh, orc, *BEAM_MODELS[0])
    p = wh.DecoderParams(prompt=[5, 6, 7], beam_size=5, max_tokens=12, no_fallback=True)
    free = ref.decode(enc, p)
    for eot in (free[4], free[6]):
        print(f"eot {eot}", flush=True)
        ref.set_eot(eot)
        dec.set_vocabulary(eot)
        assert dec.decode_tokens(enc, p) == ref.decode(enc, p)
    dec.close()


def test_beam_streak_stop_vs_oracle(wh, orc, gpu):
    """A decoder whose token T always wins: the first beam's streak of T
    (prompt included) passes 20 and the search stops (decoder.go:703-718)."""
    T = 77
    tensors, meta = forced_repeat_model(wh, T)
    dec, ref = wh.HIPDecoder(tensors, meta), orc.OracleModel(tensors, meta)
    dec.set_vocabulary(599)
    ref.set_eot(599)
    enc = wh.synth.encoder_output("repeat", 64, enc_len=40)
    for prompt, mt in (([1, 2] + [T] * 20, 5), ([1, 2], 30), ([4], 25)):
        print(f"streak prompt {len(prompt)}", flush=True)
        p = wh.DecoderParams(prompt=prompt, beam_size=5, max_tokens=mt, no_fallback=True)
        want = ref.decode(enc, p)
        assert dec.decode_tokens(enc, p) == want
    dec.close()


def test_beam_context_overflow_fails_like_oracle(wh, orc, gpu):
    """Hypotheses that read an already rewritten parent grow by more than one
    token per step; with a 12-position context one reaches the last position and
    the next forward fails in both (decoder.go:751-753), or both finish."""
    dec, ref, enc = _setup(wh, orc, "bctx", 8, (700, 64, 2, 1, 12), 30)
    p = wh.DecoderParams(prompt=[3, 4, 5], beam_size=5, max_tokens=0, no_fallback=True)
    try:
        want = ref.decode(enc, p)
    except RuntimeError as e:
        assert "context length" in str(e)
        with pytest.raises(wh.native.WhError, match="context length"):
            dec.decode_tokens(enc, p)
    else:
        assert dec.decode_tokens(enc, p) == want
    dec.close()


def test_batch_per_stream_params(wh, orc, gpu):
    """wh_decode_batch samples every stream with its own temperature,
    SuppressNST and NoSpeechThold: each equals wh_decode of that stream alone."""
    T = 77
    tensors, meta = forced_repeat_model(wh, T, dims=(600, 64, 2, 1, 64), name="pstream", gap=8.0)
    dec, ref = wh.HIPDecoder(tensors, meta), orc.OracleModel(tensors, meta)
    dec.set_vocabulary(T)
    ref.set_eot(T)
    encs = [wh.synth.encoder_output("pstream", 64, stream=i, enc_len=40) for i in range(4)]
    params = [wh.DecoderParams(prompt=[1, 2, 3], max_tokens=12, no_fallback=True),
              wh.DecoderParams(prompt=[1, 2, 3], max_tokens=12, no_fallback=True, suppress_nst=True,
                               no_speech_thold=-1e9),
              wh.DecoderParams(prompt=[4, 5], max_tokens=12, no_fallback=True, suppress_nst=True,
                               no_speech_thold=1e9, temperature=0.5),
              wh.DecoderParams(prompt=[6], max_tokens=12, no_fallback=True, suppress_nst=True,
                               no_speech_thold=-1e9, temperature=2.0)]
    got = dec.decode_batch(encs, params)
    for i in range(4):
        print(f"stream {i}", flush=True)
        assert got[i] == ref.decode(encs[i], params[i]), i
    # the suppressed streams really took the branch: EOT (= T, the top token) never appears
    assert T not in got[1][3:] and T not in got[3][1:]
    assert got[0][3] == T
    dec.close()


def test_batch_rejects_beam(wh, orc, gpu):
    dec, _, enc = _setup(wh, orc, *BEAM_MODELS[0])
    p = wh.DecoderParams(prompt=[5], beam_size=3, max_tokens=2, no_fallback=True)
    with pytest.raises(wh.native.WhError) as e:
        dec.decode_batch([enc, enc], [p, p])
    assert e.value.code == wh.native.WH_ERR_UNSUPPORTED
    dec.close()


@pytest.mark.parametrize("prompt", [[1], [1, 2, 3]])
def test_suppress_nst_greedy_vs_oracle(wh, orc, gpu, prompt):
    """SuppressNST (decoder.go:1016-1034): EOT is the top token at every step and
    its penalised logit is below -NoSpeechThold, so the best other token is taken
    instead. Prompt [1] runs its first step on the multi-kernel path and the rest
    in the persistent kernel; [1, 2, 3] runs every step persistently."""
    T = 77
    tensors, meta = forced_repeat_model(wh, T, name="supp", gap=8.0)
    dec, ref = wh.HIPDecoder(tensors, meta), orc.OracleModel(tensors, meta)
    dec.set_vocabulary(T)
    ref.set_eot(T)
    enc = wh.synth.encoder_output("supp", 64, enc_len=40)
    p = wh.DecoderParams(prompt=prompt, max_tokens=16, no_fallback=True, suppress_nst=True, no_speech_thold=-1e9)
    want = ref.decode(enc, p)
    assert T not in want[len(prompt):] and len(want) == len(prompt) + 16
    assert dec.decode_tokens(enc, p) == want
    # without the suppression EOT ends the decode at once
    p.suppress_nst = False
    assert dec.decode_tokens(enc, p) == ref.decode(enc, p) == prompt + [T]
    dec.close()


@contextlib.contextmanager
def batch_path(on):
    """The batched persistent forward is chosen when a sequence is created
    (WHISPER_HIP_BATCH, on unless 0)."""
    old = os.environ.get("WHISPER_HIP_BATCH")
    os.environ["WHISPER_HIP_BATCH"] = "1" if on else "0"
    try:
        yield
    finally:
        if old is None:
            del os.environ["WHISPER_HIP_BATCH"]
        else:
            os.environ["WHISPER_HIP_BATCH"] = old


BATCH_MODELS = [
    ("pb51", 7, (1200, 128, 2, 2, 48), 100),
    ("pb80", 8, (2000, 192, 3, 2, 64), 300),
    ("pb40", 2, (900, 128, 2, 1, 64), 1500),
    ("pb41", 3, (1500, 256, 4, 2, 64), 513),
    ("pb50", 6, (1000, 128, 2, 2, 64), 130),
]


@pytest.mark.parametrize("name,qtype,dims,enc_len", BATCH_MODELS)
@pytest.mark.parametrize("S", [2, 5, 8, 16])
def test_batched_forward_vs_multikernel_and_oracle(wh, orc, gpu, name, qtype, dims, enc_len, S):
    """The batched persistent forward (one launch per step for 2..16 states) gives
    the multi-kernel path's logits (same arithmetic, another summation order) and
    the oracle's, for states at position 0 (its own barrier) and past it."""
    print(f"batched {name} S={S}", flush=True)
    tensors, meta = wh.synth.make_decoder(name, qtype, dims=dims)
    encs = [wh.synth.encoder_output(name, dims[1], stream=i, enc_len=enc_len) for i in range(S)]
    dec = wh.HIPDecoder(tensors, meta)
    ref = orc.OracleModel(tensors, meta)
    prompts = [[1 + i] if i % 3 == 0 else list(range(2, 4 + i)) for i in range(S)]
    seqs = {}
    for on in (True, False):
        with batch_path(on):
            seqs[on] = dec.sequence(encs)
        for i, p in enumerate(prompts):
            seqs[on].set_tokens(i, p)
    seqs[True].set_profiling(True)
    states = [ref.state(p) for p in prompts]
    for step in range(3):
        ids_b, lg_b = seqs[True].step_greedy(logits=True)
        ids_m, lg_m = seqs[False].step_greedy(logits=True)
        for i in range(S):
            want = states[i].forward(encs[i])
            assert rel_err(lg_b[i], want) < 1e-3, (name, S, step, i)
            assert rel_err(lg_b[i], lg_m[i]) < 2e-5, (name, S, step, i)
            states[i].push(ids_b[i])
        assert ids_b == ids_m, (name, S, step)
    prof = seqs[True].profile()
    assert prof.get("forward_batch", (0, 0, 0))[1] == 3, prof
    for sq in seqs.values():
        sq.close()
    dec.close()


def test_last_decode_steps(wh, orc, gpu):
    """wh_last_decode_steps counts token-loop iterations: for greedy decoding the
    generated tokens, for beam search the steps even where the best hypothesis
    grew by more than one token per step."""
    dec, ref, enc = _setup(wh, orc, *BEAM_MODELS[0])
    p = wh.DecoderParams(prompt=[5, 6, 7], max_tokens=9, no_fallback=True)
    got = dec.decode_tokens(enc, p)
    assert dec.last_decode_steps() == len(got) - 3 == 9
    p = wh.DecoderParams(prompt=[5, 6, 7], beam_size=5, max_tokens=12, no_fallback=True)
    got = dec.decode_tokens(enc, p)
    assert got == ref.decode(enc, p)
    assert dec.last_decode_steps() == 12
    dec.close()
