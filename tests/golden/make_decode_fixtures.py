"""Writes the oracle's decode results for the full-size decode workloads as fixtures.

For each workload the synthetic model and encoder outputs are regenerated from
their seeds (whisper.go_amd/synth.py), so the fixture holds only results:

* decode_tiny.en_q8_0_greedy64.json      tiny.en Q8_0, greedy, 64 tokens
* decode_large-v3_q8_0_greedy224.json    large-v3 Q8_0, greedy, 224 tokens
* decode_small_q5_1_beam5_128.json       small Q5_1, beam 5, 128 steps
* decode_large-v3_q4_1_streams16.json    large-v3 Q4_1, 16 streams x 128 tokens,
                                         prompts of 4..224 tokens

Greedy records hold the full token sequence (prompt + generated), the margin
between the best and second-best penalised logit at every step (a step whose
margin is below the logits' error bound is "fragile": a token difference there
is not a parity failure by itself), and the first step's largest logits. Beam
records hold the first beam's tokens after 8, 16, 32, 64 and 128 steps, every
final beam, and the per-step margin of the prune (smallest gap between two
different normalised scores at the selection boundary).

Run from the repository root (the oracle must be built: make -C oracle):
    python tests/golden/make_decode_fixtures.py [--threads 8] [--only NAME]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import __graft_entry__  # noqa: E402
from oracle import oracle as orc  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def oracle_model(tensors, meta, threads):
    ref = orc.OracleModel(tensors, meta, dot_variant=1, threads=threads)
    ref.set_forward_threads(threads)
    return ref


def greedy_record(wh, ref, enc, prompt, max_tokens, check_decode=False):
    """The greedy loop of decoder.go:441-485 stepped through the oracle's forward,
    penalty and selection, so every step's margin (best minus second-best
    penalised logit) comes from the forward that chose its token. check_decode
    also runs the oracle's own decode loop and requires the same tokens."""
    st = ref.state(prompt)
    st.prepare_cross(enc)
    toks, margins, first = list(prompt), [], None
    mt = max_tokens if max_tokens > 0 else ref.n_ctx
    mt = max(0, min(mt, ref.n_ctx - len(prompt)))
    prev, streak = -1, 0
    for _ in range(mt):
        logits = st.forward(enc)
        if first is None:
            top = np.argsort(-logits, kind="stable")[:8]
            first = {"top_ids": [int(t) for t in top], "top_values": [float(logits[t]) for t in top],
                     "max_abs": float(np.max(np.abs(logits)))}
        cur = orc.repetition_penalty(logits, np.array(toks, np.int32))
        nxt = int(orc.sample_greedy(cur, 1.0, eot=ref.eot))
        srt = np.sort(cur)[::-1]
        margins.append(float(srt[0] - srt[1]))
        toks.append(nxt)
        st.push(nxt)
        if nxt == ref.eot:
            break
        streak = streak + 1 if nxt == prev else 1
        prev = nxt
        if streak > 20:
            break
    if check_decode:
        p = wh.DecoderParams(prompt=list(prompt), max_tokens=max_tokens, no_fallback=True)
        assert ref.decode(enc, p) == toks, "stepping disagrees with the oracle's decode loop"
    return {"prompt": list(prompt), "tokens": toks, "margins": margins, "first_logits": first}


def make_greedy(wh, name, config, qtype, n_tok, threads):
    tensors, meta = wh.synth.make_decoder(config, qtype)
    enc = wh.synth.encoder_output(config, meta["n_state"], stream=0)
    ref = oracle_model(tensors, meta, threads)
    rec = greedy_record(wh, ref, enc, wh.synth.SOT_EN_TRANSCRIBE, n_tok, check_decode=config == "tiny.en")
    return {"workload": name, "config": config, "qtype": qtype, "max_tokens": n_tok, "encoder_stream": 0, **rec}


def make_beam(wh, name, config, qtype, beam, n_tok, threads):
    tensors, meta = wh.synth.make_decoder(config, qtype)
    enc = wh.synth.encoder_output(config, meta["n_state"], stream=0)
    ref = oracle_model(tensors, meta, threads)
    prompt = list(wh.synth.SOT_EN_TRANSCRIBE)
    p = wh.DecoderParams(prompt=prompt, beam_size=beam, max_tokens=n_tok, no_fallback=True)
    beams, margins = ref.beam_run(enc, p, margins=True)
    toks = beams[0][0]
    # the first beam after k steps: a run of k steps compares exactly while every
    # prune up to step k is far from a reorder
    checkpoints = {}
    for k in (8, 16, 32, 64):
        pk = wh.DecoderParams(prompt=prompt, beam_size=beam, max_tokens=k, no_fallback=True)
        checkpoints[str(k)] = ref.decode(enc, pk)
    checkpoints[str(n_tok)] = toks
    return {"workload": name, "config": config, "qtype": qtype, "beam_size": beam, "max_tokens": n_tok,
            "encoder_stream": 0, "prompt": prompt, "tokens": toks, "checkpoints": checkpoints,
            "beams": [{"tokens": b[0], "score": b[1]} for b in beams], "margins": margins}


def make_streams(wh, name, config, qtype, n_streams, n_tok, threads):
    tensors, meta = wh.synth.make_decoder(config, qtype)
    ref = oracle_model(tensors, meta, threads)
    prompts = wh.synth.stream_prompts(n_streams)
    streams = []
    for i, prompt in enumerate(prompts):
        t0 = time.time()
        enc = wh.synth.encoder_output(config, meta["n_state"], stream=i)
        rec = greedy_record(wh, ref, enc, prompt, n_tok)
        streams.append({"encoder_stream": i, **rec})
        log(f"  stream {i}: prompt {len(prompt)}, {len(rec['tokens']) - len(prompt)} tokens, "
            f"{time.time() - t0:.0f}s")
    return {"workload": name, "config": config, "qtype": qtype, "max_tokens": n_tok, "streams": streams}


JOBS = {
    "decode_tiny.en_q8_0_greedy64": lambda wh, t: make_greedy(wh, "tiny.en Q8_0 greedy x64", "tiny.en", 8, 64, t),
    "decode_large-v3_q8_0_greedy224": lambda wh, t: make_greedy(wh, "large-v3 Q8_0 greedy x224", "large-v3", 8,
                                                                224, t),
    "decode_small_q5_1_beam5_128": lambda wh, t: make_beam(wh, "small Q5_1 beam 5 x128", "small", 7, 5, 128, t),
    "decode_large-v3_q4_1_streams16": lambda wh, t: make_streams(wh, "large-v3 Q4_1 16 streams x128", "large-v3", 3,
                                                                 16, 128, t),
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--only", default=None)
    a = ap.parse_args()
    wh = __graft_entry__.load_package()
    for name, job in JOBS.items():
        if a.only and a.only != name:
            continue
        t0 = time.time()
        log(f"{name} ...")
        rec = job(wh, a.threads)
        path = os.path.join(HERE, name + ".json")
        with open(path, "w") as f:
            json.dump(rec, f, separators=(",", ":"))
            f.write("\n")
        log(f"{name}: {time.time() - t0:.0f}s -> {os.path.relpath(path, ROOT)}")


if __name__ == "__main__":
    main()
