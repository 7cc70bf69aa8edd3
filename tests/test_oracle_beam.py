"""The oracle's beam search and stop rules pinned against hand-derived results.

Beam pruning in the reference (internal/model/decoder.go:575-718) sorts the
candidates with Go's sort.Slice (pdqsort, not stable) and builds the next
hypotheses inside the current beam objects, popping them from the end of
reusableBeams. The expected orders and histories below were traced by hand
from those two pieces of code; none of them is computed by restating the
algorithm in the test.
"""
import numpy as np
import pytest


# ---- Go's sort.Slice (pdqsort) ------------------------------------------------

def test_go_sort_step0_pattern_hand_trace(orc):
    """25 candidates as five identical hypotheses propose them at the first beam
    step: candidate 5b + r has the score of rank r (s0 > ... > s4). Tracing
    pdqsort by hand (median-of-three pivot at 12 with no swaps, a failed partial
    insertion sort at i = 5, a partition around s2 that ends at mid = 10, then
    insertion sort of [0, 10), a second partition of [11, 25) around index 20 and
    insertion sorts of both sides) gives this permutation of (b, r)."""
    s = [-0.1, -2.0, -3.0, -4.0, -5.0]
    norm = [s[i % 5] for i in range(25)]
    _, ids = orc.go_sort_norm(norm)
    got = [(int(i) // 5, int(i) % 5) for i in ids]
    want = [(2, 0), (4, 0), (1, 0), (3, 0), (0, 0),
            (0, 1), (4, 1), (3, 1), (1, 1), (2, 1),
            (2, 2), (1, 2), (4, 2), (0, 2), (3, 2),
            (0, 3), (3, 3), (2, 3), (1, 3), (4, 3),
            (0, 4), (2, 4), (3, 4), (1, 4), (4, 4)]
    assert got == want


def test_go_sort_all_equal_is_identity(orc):
    """Equal keys: the pivot choice makes no swaps, the partial insertion sort
    finds the range sorted and returns at once."""
    for n in (13, 25, 60):
        _, ids = orc.go_sort_norm(np.zeros(n, np.float32))
        assert ids.tolist() == list(range(n))


def test_go_sort_small_is_stable(orc):
    """Up to 12 elements sort.Slice is an insertion sort that only swaps on a
    strict less: equal keys keep their input order."""
    rng = np.random.default_rng(5)
    for n in range(1, 13):
        keys = rng.integers(0, 3, n).astype(np.float32)
        _, ids = orc.go_sort_norm(keys)
        want = sorted(range(n), key=lambda i: (-keys[i], i))
        assert ids.tolist() == want


@pytest.mark.parametrize("n", [13, 24, 25, 49, 50, 51, 80, 200])
def test_go_sort_sorts(orc, n):
    """Every length and key pattern (ties, presorted, reversed, random; the
    ninther pivot from 50 elements) yields a non-increasing permutation."""
    rng = np.random.default_rng(n)
    patterns = [rng.standard_normal(n), rng.integers(0, 4, n), np.arange(n), -np.arange(n),
                np.r_[np.arange(n // 2), np.arange(n - n // 2)], np.ones(n)]
    for keys in patterns:
        keys = np.asarray(keys, np.float32)
        srt, ids = orc.go_sort_norm(keys)
        assert sorted(ids.tolist()) == list(range(n))
        assert np.array_equal(srt, keys[ids])
        assert np.all(srt[:-1] >= srt[1:])


# ---- beam search with in-place reuse -------------------------------------------

def _model(wh, orc, name, dims=(600, 64, 2, 1, 48), qtype=8):
    tensors, meta = wh.synth.make_decoder(name, qtype, dims=dims)
    enc = wh.synth.encoder_output(name, dims[1], enc_len=40)
    return tensors, meta, orc.OracleModel(tensors, meta), enc


def _top5(orc, ref, enc, prompt):
    st = ref.state(prompt)
    pen = orc.repetition_penalty(st.forward(enc), np.array(prompt, np.int32))
    return orc.topk(pen, 5, 1.0)


@pytest.mark.parametrize("prompt", [[5, 6, 7], [9]])
def test_beam_first_step_histories(wh, orc, prompt):
    """After one step from five identical hypotheses the sorted top five are the
    rank-0 candidates of beams 2, 4, 1, 3, 0 (trace above). Slot 0 reuses object
    4 with parent 2: [P, A]. Slot 1 reuses object 3 whose parent, object 4, now
    holds [P, A]: [P, A, A]. Slot 2 reuses object 2 with parent 1: [P, A]. Slot
    3 reuses object 1, parent object 3 = [P, A, A]: [P, A, A, A]. Slot 4 reuses
    object 0, its own parent, whose capacity len(P) is short: make() zeroes the
    slice and the copy onto itself keeps the zeros: [0 x len(P), A]."""
    _, _, ref, enc = _model(wh, orc, "beam1")
    tok, lp = _top5(orc, ref, enc, prompt)
    assert len(set(lp.tolist())) == 5  # distinct ranks, as the trace assumes
    A = int(tok[0])
    beams = ref.beam_run(enc, wh.DecoderParams(prompt=prompt, beam_size=5, max_tokens=1, no_fallback=True))
    P = list(prompt)
    want = [P + [A], P + [A, A], P + [A], P + [A, A, A], [0] * len(P) + [A]]
    assert [b[0] for b in beams] == want
    assert all(b[1] == np.float32(lp[0]) for b in beams)
    # Decode returns the first beam
    p = wh.DecoderParams(prompt=prompt, beam_size=5, max_tokens=1, no_fallback=True)
    assert ref.decode(enc, p) == P + [A]


def test_beam_all_eot_stops(wh, orc):
    """With EOT set to the step's best token every hypothesis ends in EOT after
    the first step and the search stops (decoder.go:690-700), whatever the
    token budget: the result is the first beam, [P, EOT]."""
    _, _, ref, enc = _model(wh, orc, "beameot")
    prompt = [3, 4]
    tok, _ = _top5(orc, ref, enc, prompt)
    ref.set_eot(int(tok[0]))
    p = wh.DecoderParams(prompt=prompt, beam_size=5, max_tokens=10, no_fallback=True)
    assert ref.decode(enc, p) == prompt + [int(tok[0])]
    beams = ref.beam_run(enc, p)
    assert all(b[0][-1] == int(tok[0]) for b in beams)


def _forced_repeat_model(wh, orc, T):
    """Logits fixed by the final LayerNorm's bias: token T at 100, every other
    token O(0.1), so T wins every step even after the repetition penalty of 2
    per occurrence has taken 40 from it (tests/models.py)."""
    from models import forced_repeat_model

    return forced_repeat_model(wh, T)


def test_greedy_streak_stop(wh, orc):
    """decoder.go:474-484: the greedy loop stops once the same token has been
    generated more than 20 times in a row (the prompt does not count), with EOT
    out of reach."""
    T = 77
    tensors, meta = _forced_repeat_model(wh, orc, T)
    ref = orc.OracleModel(tensors, meta)
    ref.set_eot(-1)
    enc = wh.synth.encoder_output("repeat", 64, enc_len=40)
    prompt = [1, 2, 3]
    p = wh.DecoderParams(prompt=prompt, max_tokens=40, no_fallback=True)
    assert ref.decode(enc, p) == prompt + [T] * 21


def test_beam_streak_stop(wh, orc):
    """decoder.go:703-718: the beam loop stops when the first beam's last token
    repeats more than 20 times, counting the prompt. The prompt ends in 20
    copies of T; after the first step beam 0 is [P, T] (the first-step pattern
    above), a streak of 21, so the search ends there instead of running the
    five steps it may."""
    T = 77
    tensors, meta = _forced_repeat_model(wh, orc, T)
    ref = orc.OracleModel(tensors, meta)
    ref.set_eot(-1)
    enc = wh.synth.encoder_output("repeat", 64, enc_len=40)
    prompt = [1, 2] + [T] * 20
    tok, lp = _top5(orc, ref, enc, prompt)
    assert int(tok[0]) == T and len(set(lp.tolist())) == 5
    p = wh.DecoderParams(prompt=prompt, beam_size=5, max_tokens=5, no_fallback=True)
    assert ref.decode(enc, p) == prompt + [T]
    # a shorter run of T in the prompt does not stop it
    p2 = wh.DecoderParams(prompt=[1, 2] + [T] * 5, beam_size=5, max_tokens=3, no_fallback=True)
    assert len(ref.decode(enc, p2)) > len(p2.prompt) + 1
