"""Decode throughput of the whisper decoder token loop on one MI355X.

Default workload: large-v3 decoder (d=1280, 32 layers, 20 heads, V=51866,
n_text_ctx 448), seeded N(0,0.02) weights quantised to Q8_0 with the
cmd/quantize rule, synthetic 1500x1280 N(0,1) encoder output, greedy decoding
at batch 1 from the SOT/en/transcribe prompt. A step is one decoded token
(forward + repetition penalty + argmax on device; only the id crosses PCIe).
`--warmup` steps (the first includes nothing extra: the cross K/V are built
when the sequence is created) run untimed, then `--steps` steps are timed.

Also reported:
* roofline: the dominant kernel class measured with HIP events around every
  launch in a separate profiled pass of the same steps; achieved = algorithmic
  bytes / kernel time, against 8 TB/s.
* cpu_baseline: the oracle (a C restatement of the Go decoder) on the host
  cores, one thread (the reference's batch-1 GEMV is single-threaded), on a
  bounded sample of the same workload.

`--workload beam5|streams16` instead times one of the batched workloads (beam 5
over the small decoder in Q5_1; 16 large-v3 Q4_1 streams) as one Decode call;
`--workload encoder` times the encoder forward of one 30 s window.
`--gemv` instead runs the standalone quantised-GEMV microbench (rows x cols at
batch 1 and 5 for each format, rotating over >= 1 GiB of distinct copies;
back-to-back launches replayed from a HIP graph, time per launch).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
import __graft_entry__  # noqa: E402

HBM_PEAK_GBS = 8000.0
QNAMES = {"Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or the platform string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or platform.machine()


def host_cores():
    """CPUs this process may run on (its affinity share, not the machine's count)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def prefix_match(a, b):
    """(equal, n): whether the first n = min(len(a), len(b)) tokens agree."""
    n = min(len(a), len(b))
    return list(a[:n]) == list(b[:n]), n


def cpu_baseline(wh, tensors, meta, enc, prompt, n_tokens, gpu_tokens):
    from oracle import oracle as orc  # the oracle, timed as the CPU baseline

    threads = min(16, host_cores())
    t0 = time.time()
    ref = orc.OracleModel(tensors, meta, dot_variant=1, threads=threads)
    st = ref.state(prompt)
    st.prepare_cross(enc)  # the one-time cross K/V precompute, multi-threaded, untimed
    t_cross = time.time() - t0
    toks = list(prompt)
    margins = []
    t1 = time.perf_counter()
    for _ in range(n_tokens):
        logits = st.forward(enc)
        cur = orc.repetition_penalty(logits, np.array(toks, np.int32))
        nxt = orc.sample_greedy(cur, 1.0, eot=50256)
        toks.append(int(nxt))
        st.push(nxt)
        top2 = np.partition(cur, -2)[-2:]
        margins.append(float(abs(top2[1] - top2[0]) / max(float(np.max(np.abs(cur))), 1e-30)))
    dt = time.perf_counter() - t1
    gen = toks[len(prompt):]
    match, n = prefix_match(gen, gpu_tokens)
    return {"value": n_tokens / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "label": "restatement, not Go: the C oracle restating the Go decoder (no Go toolchain in the image)",
            "cpu_model": cpu_model(), "host_cores": host_cores(),
            "sample": f"{n_tokens} greedy steps of the same workload after the cross K/V precompute "
                      f"({t_cross:.1f}s on {threads} threads, untimed); the batch-1 GEMV is single-threaded "
                      f"as in the reference",
            "tokens_match_gpu": match, "tokens_compared": n,
            "min_top1_top2_margin": round(min(margins), 6) if margins else None,
            "fragile_steps": sum(m < 1e-5 for m in margins),
            "margin_note": "(top-1 - top-2) / max |logit| of each sampled step's penalised logits; a step is "
                           "fragile below 1e-5, where fp32 reassociation could flip the argmax"}


def generate_n(seq, n):
    """n greedy tokens of stream 0; generate() stops early on the reference's
    stop rules (EOT, repeats), so call it again until n tokens exist."""
    out = []
    while len(out) < n:
        got = seq.generate(n - len(out))
        if not got:
            raise SystemExit("bench: generate made no progress")
        out += got
    return out


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_persistent_large-v3_q8_0.md")


def measured_traffic(config, qtype, persistent):
    """HBM bytes per token of the persistent kernel on large-v3 Q8_0, from the
    committed rocprofv3 --pmc summary (FETCH_SIZE x 2 + WRITE_SIZE x 1, scaled
    by a device-to-device copy of known size), or None for other workloads."""
    if not (persistent and config == "large-v3" and qtype == "Q8_0") or not os.path.exists(TRAFFIC_PROFILE):
        return None
    with open(TRAFFIC_PROFILE) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_token:"):
                return int(line.split(":")[1])
    return None


def copy_calibration(wh, mib):
    """Device-to-device copies of a known size: their FETCH_SIZE / WRITE_SIZE in
    a rocprofv3 --pmc run give the scale factor for the decode kernel's counters."""
    n = mib << 20
    src, dst = wh.native.DevBuf(n), wh.native.DevBuf(n)
    for _ in range(2):
        wh.native.check(wh.native.lib().wh_memcpy(dst.ptr, src.ptr, n, 2))
    log(f"bench: copy calibration: 2 x {n} bytes device to device")
    src.free()
    dst.free()


def run_decode(args):
    wh = __graft_entry__.load_package()
    if wh.native.device_count() < 1:
        raise SystemExit("bench: no GPU visible")
    if args.copy_mib > 0:
        copy_calibration(wh, args.copy_mib)
    qtype = QNAMES[args.qtype]
    t0 = time.time()
    tensors, meta = wh.synth.make_decoder(args.config, qtype)
    d = meta["n_state"]
    enc = wh.synth.encoder_output(args.config, d, stream=0)
    prompt = list(wh.synth.SOT_EN_TRANSCRIBE)
    wbytes = wh.synth.weight_bytes_per_token(tensors)
    log(f"bench: model {args.config} {args.qtype} generated in {time.time() - t0:.1f}s, {wbytes} weight B/token")
    total = args.warmup + args.steps
    if len(prompt) + total > meta["n_ctx"]:
        raise SystemExit(f"bench: {total} steps exceed n_text_ctx {meta['n_ctx']}")
    t0 = time.time()
    dec = wh.HIPDecoder(tensors, meta, device=0)
    if dec.weight_bytes != wbytes:
        raise SystemExit(f"bench: device weight bytes {dec.weight_bytes} != {wbytes}")
    log(f"bench: weights uploaded in {time.time() - t0:.2f}s")
    # first token from the host encoder output: sequence creation (encoder output
    # upload + the cross K/V of every layer) and the first step
    t1 = time.perf_counter()
    seq = dec.sequence([enc])
    seq.set_tokens(0, prompt)
    setup_ms = (time.perf_counter() - t1) * 1e3
    persistent = seq.persistent[0]
    log(f"bench: cross K/V in {setup_ms:.1f} ms, persistent kernel: {persistent}")
    t1 = time.perf_counter()
    tokens = generate_n(seq, 1)
    first_ms = (time.perf_counter() - t1) * 1e3
    t1 = time.perf_counter()
    tokens += generate_n(seq, args.warmup - 1) if args.warmup > 1 else []
    t_warm_ms = (time.perf_counter() - t1) * 1e3
    # timed region: HIP events around each launch give the kernel's own time
    seq.set_profiling(True)
    launches0 = seq.persistent[1]
    t1 = time.perf_counter()
    timed = generate_n(seq, args.steps)
    dt = time.perf_counter() - t1
    prof = seq.profile()
    launches = seq.persistent[1] - launches0
    seq.set_profiling(False)
    tokens += timed
    seq.close()
    log(f"bench: {args.steps} steps in {dt * 1e3:.1f} ms ({launches} persistent launches)")
    kern_ms = {k: v[0] for k, v in prof.items()}
    dom = max(kern_ms, key=kern_ms.get)
    dms, dcount, dbytes = prof[dom]
    achieved = dbytes / (dms * 1e-3) / 1e9 if dms > 0 else 0.0
    value = args.steps / dt
    tpt = measured_traffic(args.config, args.qtype, persistent)
    traffic = round(tpt * args.steps / max(dcount, 1)) if tpt and dom == "decode_persistent" else None
    out = {
        "metric": "decode tokens/s (large-v3 Q8_0, bs=1)" if args.config == "large-v3" and args.qtype == "Q8_0"
        else f"decode tokens/s ({args.config} {args.qtype}, bs=1)",
        "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"whisper {args.config} decoder, {args.qtype} weights, greedy, batch 1, "
                               f"1500x{d} synthetic encoder output", "global_batch": 1,
                   "prompt": prompt, "steps_timed": args.steps, "weights": args.qtype},
        "path": "persistent" if persistent else "multi-kernel",
        "first_token_ms": round(first_ms, 3),
        "sequence_setup_ms": round(setup_ms, 3),
        "first_token_with_cross_kv_ms": round(setup_ms + first_ms, 3),
        "end_to_end_ms": round(setup_ms + first_ms + (t_warm_ms + dt * 1e3), 3),
        "weight_bytes_per_token": wbytes,
        "weight_roofline_frac": round(wbytes * value / (HBM_PEAK_GBS * 1e9), 4),
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "launches": dcount, "avg_launch_us": round(dms * 1e3 / max(dcount, 1), 3),
                     "bytes_per_launch": round(dbytes / max(dcount, 1)), "traffic": traffic,
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE of this launch shape, "
                                       "profiles/decode_persistent_large-v3_q8_0.md" if traffic else None},
        "kernel_ms_per_step": {k: round(v / args.steps, 4) for k, v in kern_ms.items()},
        "stopped_at_step": next((i + 1 for i, t in enumerate(tokens) if t == dec.eot), None),
    }
    if args.multikernel_steps > 0:
        # the same tokens through one launch per kernel (the persistent kernel off)
        os.environ["WHISPER_HIP_PERSISTENT"] = "0"
        s0 = dec.sequence([enc])
        del os.environ["WHISPER_HIP_PERSISTENT"]
        s0.set_tokens(0, prompt)
        mk = [s0.step_greedy()[0] for _ in range(4)]
        t1 = time.perf_counter()
        mk += [s0.step_greedy()[0] for _ in range(args.multikernel_steps)]
        mdt = time.perf_counter() - t1
        s0.close()
        match, n = prefix_match(mk, tokens)
        out["multikernel"] = {"tokens_per_s": round(args.multikernel_steps / mdt, 2),
                              "tokens_match": match, "tokens_compared": n}
    dec.close()
    if args.cpu_tokens > 0:
        log("bench: cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(wh, tensors, meta, enc, prompt, args.cpu_tokens, tokens)
    print(json.dumps(out), flush=True)


def run_batched(args):
    """The two batched workloads: beam 5 over the small decoder in Q5_1 (128 steps)
    and 16 independent large-v3 Q4_1 streams with prompts of 4..224 tokens (128
    greedy tokens each). Each is one Decode call (decode_tokens, decode_batch) timed
    end to end, cross K/V precompute and host bookkeeping included; a short call of
    the same kind runs first, untimed."""
    wh = __graft_entry__.load_package()
    if wh.native.device_count() < 1:
        raise SystemExit("bench: no GPU visible")
    prompt0 = list(wh.synth.SOT_EN_TRANSCRIBE)
    if args.workload == "beam5":
        config, qname, beam, n_tok = "small", "Q5_1", 5, 128
        tensors, meta = wh.synth.make_decoder(config, QNAMES[qname])
        d = meta["n_state"]
        enc = wh.synth.encoder_output(config, d, stream=0)
        dec = wh.HIPDecoder(tensors, meta, device=0)
        dec.decode_tokens(enc, wh.DecoderParams(prompt=prompt0, beam_size=beam, max_tokens=4, no_fallback=True))
        p = wh.DecoderParams(prompt=prompt0, beam_size=beam, max_tokens=n_tok, no_fallback=True)
        t1 = time.perf_counter()
        toks = dec.decode_tokens(enc, p)
        dt = time.perf_counter() - t1
        # token-loop iterations: under the reference's in-place beam reuse the best
        # hypothesis can grow by more than one token per step
        steps = dec.last_decode_steps()
        wbytes = wh.synth.weight_bytes_per_token(tensors)
        out = {"metric": "beam-5 decode steps/s (small Q5_1)", "value": round(steps / dt, 2), "unit": "steps/s",
               "n_gpus": 1, "steps": steps, "higher_is_better": True, "ms_per_step": round(dt * 1e3 / max(steps, 1), 4),
               "hypothesis_tokens_per_s": round(beam * steps / dt, 2), "best_hypothesis_tokens": len(toks) - len(prompt0),
               "dtype": "f32", "data": "synthetic",
               "weight_bytes_per_step": wbytes,
               "weight_roofline_frac": round(wbytes * steps / dt / (HBM_PEAK_GBS * 1e9), 4),
               "config": {"workload": f"whisper {config} decoder, {qname} weights, beam {beam}, {n_tok} tokens, "
                                      f"1500x{d} synthetic encoder output, one Decode call", "global_batch": beam}}
    else:
        config, qname, S, n_tok = "large-v3", "Q4_1", 16, 128
        tensors, meta = wh.synth.make_decoder(config, QNAMES[qname])
        d = meta["n_state"]
        encs = [wh.synth.encoder_output(config, d, stream=i) for i in range(S)]
        prompts = wh.synth.stream_prompts(S)
        lens = np.array([len(p) for p in prompts])
        dec = wh.HIPDecoder(tensors, meta, device=0)
        dec.decode_batch(encs[:2], [wh.DecoderParams(prompt=prompts[i], max_tokens=4, no_fallback=True)
                                    for i in range(2)])
        params = [wh.DecoderParams(prompt=prompts[i], max_tokens=n_tok, no_fallback=True) for i in range(S)]
        t1 = time.perf_counter()
        got = dec.decode_batch(encs, params)
        dt = time.perf_counter() - t1
        gen = sum(len(g) - len(prompts[i]) for i, g in enumerate(got))
        steps = dec.last_decode_steps()
        out = {"metric": "16-stream batched decode tokens/s (large-v3 Q4_1)", "value": round(gen / dt, 2),
               "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True, "tokens": gen,
               "steps": steps, "ms_per_step": round(dt * 1e3 / max(steps, 1), 4), "dtype": "f32", "data": "synthetic",
               "config": {"workload": f"whisper {config} decoder, {qname} weights, {S} streams, prompts "
                                      f"{int(lens.min())}..{int(lens.max())} tokens, {n_tok} greedy tokens each, "
                                      f"1500x{d} synthetic encoder outputs, one batched Decode call",
                          "global_batch": S}}
    dec.close()
    print(json.dumps(out), flush=True)


def encoder_flops(n_mels, d, n_layer, T):
    """Multiply-add FLOPs (2 per MAC) of one encode of T mel frames: conv1
    (3 n_mels -> d per frame), conv2 (3 d -> d per output frame, stride 2), and
    per block the q, k, v, o projections (4 d^2), the MLP (8 d^2) and attention
    (scores and weights . V, 2 T'^2 d) over T' = (T + 1) / 2 frames."""
    tp = (T + 1) // 2
    conv = 2 * T * d * 3 * n_mels + 2 * tp * d * 3 * d
    block = 2 * tp * 12 * d * d + 2 * 2 * tp * tp * d
    return conv + n_layer * block


def run_encoder(args):
    """The encoder forward (internal/model/encoder.go:265-338) of one 30 s window,
    3000 mel frames -> 1500 rows, on the large-v3 encoder with seeded weights
    quantised with the cmd/quantize rule. A step is one encode with the mel and
    the output resident in HBM (wh_encode_device); the host-buffer call
    (wh_encode, PCIe copies included) is timed beside it."""
    wh = __graft_entry__.load_package()
    if wh.native.device_count() < 1:
        raise SystemExit("bench: no GPU visible")
    config, qname = args.config, args.qtype
    M, d, H, L, ctx = wh.synth.ENC_CONFIGS[config]
    T = 2 * ctx
    tensors, meta = wh.synth.make_encoder(config, QNAMES[qname])
    mel = wh.synth.mel_input(config, M, T=T)
    enc = wh.HIPEncoder(tensors, meta, device=0)
    dmel, dout = wh.native.DevBuf.from_array(mel), wh.native.DevBuf(ctx * d * 4)
    steps, warm = args.encoder_steps, 2
    for _ in range(warm):
        enc.encode_device(dmel.ptr.value, M, T, dout.ptr.value, ctx)
    t0 = time.perf_counter()
    for _ in range(steps):
        enc.encode_device(dmel.ptr.value, M, T, dout.ptr.value, ctx)
    dt = (time.perf_counter() - t0) / steps
    got = dout.download((ctx, d), np.float32)
    t1 = time.perf_counter()
    host = enc.encode(mel)
    dt_host = time.perf_counter() - t1
    flops = encoder_flops(M, d, L, T)
    tflops = flops / dt / 1e12
    peak = 157.3
    out = {"metric": f"encoder windows/s ({config} {qname}, 30 s window)", "value": round(1.0 / dt, 3),
           "unit": "windows/s", "n_gpus": 1, "steps": steps, "warmup": warm, "ms_per_step": round(dt * 1e3, 3),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic",
           "config": {"workload": f"whisper {config} encoder, {qname} weights, {M}x{T} synthetic log-mel "
                                  f"-> {ctx}x{d}, mel and output in HBM", "global_batch": 1},
           "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                        "frac": round(tflops / peak, 4), "traffic": None,
                        "scope": "whole encode (every kernel of the forward): algorithmic FLOPs / step time"},
           "flops_per_step": flops,
           "host_buffers_ms": round(dt_host * 1e3, 3),
           "device_equals_host_path": bool(np.array_equal(got, host))}
    dmel.free()
    dout.free()
    enc.close()
    if args.cpu_tokens > 0:
        from oracle import oracle as orc  # the oracle, timed as the CPU baseline

        threads = min(16, host_cores())
        n_blk = 1
        sub, smeta = wh.synth.make_encoder(config, QNAMES[qname], dims=(M, d, H, n_blk, ctx))
        ref = orc.OracleEncoder(sub, smeta, threads=threads)
        t2 = time.perf_counter()
        ref.encode(mel)
        dt_cpu = (time.perf_counter() - t2) * flops / encoder_flops(M, d, n_blk, T)
        out["cpu_baseline"] = {"value": round(1.0 / dt_cpu, 5), "unit": "windows/s", "cores": threads,
                               "kind": "port",
                               "label": "restatement, not Go: the C oracle restating the Go encoder",
                               "cpu_model": cpu_model(), "host_cores": host_cores(),
                               "sample": f"conv stem + {n_blk} of {L} blocks over the full {T} frames, "
                                         f"timed and scaled to the whole encoder by FLOPs"}
    print(json.dumps(out), flush=True)


class HipGraphs:
    """Stream capture into a HIP graph through the HIP runtime the library
    already loaded (the microbench's launch loop, replayed without Python)."""

    def __init__(self):
        import ctypes as C
        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        if path is None:
            raise RuntimeError("libamdhip64 is not loaded")
        self.C = C
        self.h = C.CDLL(path)
        for n in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
                  "hipGraphExecDestroy", "hipGraphDestroy"):
            getattr(self.h, n).restype = C.c_int
        self.h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        self.h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        self.h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
        self.h.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipGraphExecDestroy.argtypes = [C.c_void_p]
        self.h.hipGraphDestroy.argtypes = [C.c_void_p]

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: hipError {rc}")

    def capture(self, stream, issue):
        C = self.C
        self._ok(self.h.hipStreamBeginCapture(stream, 2), "hipStreamBeginCapture")  # relaxed mode
        try:
            rcs = issue()
        finally:
            g = C.c_void_p()
            self._ok(self.h.hipStreamEndCapture(stream, C.byref(g)), "hipStreamEndCapture")
        if any(rcs):
            raise RuntimeError(f"launch during capture returned {set(rcs)}")
        ex = C.c_void_p()
        self._ok(self.h.hipGraphInstantiate(C.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        return (g, ex)

    def launch(self, graph, stream):
        self._ok(self.h.hipGraphLaunch(graph[1], stream), "hipGraphLaunch")

    def destroy(self, graph):
        self.h.hipGraphExecDestroy(graph[1])
        self.h.hipGraphDestroy(graph[0])


def run_gemv(args):
    """Standalone quantised GEMV at the large-v3 decoder shapes."""
    import ctypes as C

    wh = __graft_entry__.load_package()
    lib = wh.native.lib()
    shapes = [(1280, 1280), (5120, 1280), (1280, 5120), (51866, 1280)]
    fmts = args.gemv_formats.split(",")
    st = wh.native.Stream()
    e0, e1 = wh.native.Event(), wh.native.Event()
    hip = None if args.gemv_single else HipGraphs()
    rows_out = []
    for fmt in fmts:
        qt = QNAMES[fmt]
        for rows, cols in shapes:
            rng = np.random.default_rng(rows + cols)
            w = (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
            raw = wh.quant.quantize(qt, w)
            nbytes = raw.size
            ncopy = max(2, min(256, int(np.ceil((1 << 30) / nbytes))))
            mats = []
            for _ in range(ncopy):
                h = C.c_void_p()
                wh.native.check(lib.wh_matrix_create(qt, rows, cols, raw.ctypes.data, raw.size, 0, C.byref(h)))
                mats.append(h)
            for batch in [int(b) for b in args.gemv_batches.split(",")]:
                x = wh.native.DevBuf.from_array(rng.standard_normal((batch, cols)).astype(np.float32))
                y = wh.native.DevBuf(batch * rows * 4)
                for h in mats[:4]:
                    wh.native.check(lib.wh_gemv(h, x.ptr, batch, y.ptr, st.h))
                # back-to-back launches (rotating over the copies) captured in one HIP
                # graph, timed per graph launch: the kernel plus the gap between
                # kernels, not the rate at which Python can issue launches; median
                nlaunch = max(64, ncopy)
                times = []
                if not args.gemv_single:
                    graph = hip.capture(st.h, lambda: [lib.wh_gemv(mats[i % ncopy], x.ptr, batch, y.ptr, st.h)
                                                       for i in range(nlaunch)])
                    for rep in range(12):
                        e0.record(st)
                        hip.launch(graph, st.h)
                        e1.record(st)
                        st.sync()
                        if rep >= 2:
                            times.append(e0.elapsed_ms(e1) / nlaunch)
                    hip.destroy(graph)
                # one launch alone between its own pair of events (includes the
                # launch and event latency)
                single = []
                for i in range(32):
                    e0.record(st)
                    lib.wh_gemv(mats[i % ncopy], x.ptr, batch, y.ptr, st.h)
                    e1.record(st)
                    st.sync()
                    single.append(e0.elapsed_ms(e1))
                ms = float(np.median(times if times else single))
                gbs = nbytes / (ms * 1e-3) / 1e9
                rows_out.append({"format": fmt, "rows": rows, "cols": cols, "batch": batch, "bytes": nbytes,
                                 "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                 "us_single_launch": round(float(np.median(single)) * 1e3, 3),
                                 "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": ncopy,
                                 "timing": "graph" if times else "single"})
                log(json.dumps(rows_out[-1]))
            for h in mats:
                lib.wh_matrix_destroy(h)
    print(json.dumps({"metric": "quant-GEMV HBM GB/s as % of peak", "rows": rows_out}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=224)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="large-v3")
    ap.add_argument("--qtype", default="Q8_0", choices=sorted(QNAMES))
    ap.add_argument("--multikernel-steps", type=int, default=32,
                    help="also time this many steps with one launch per kernel (0 = skip)")
    ap.add_argument("--cpu-tokens", type=int, default=30,
                    help="oracle steps timed for cpu_baseline, about 0.4 s each (0 = skip)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first copy this many MiB device to device (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--gemv", action="store_true", help="run the standalone GEMV microbench instead")
    ap.add_argument("--workload", choices=["beam5", "streams16", "encoder"], default=None,
                    help="run another workload instead: beam 5 small Q5_1; 16 large-v3 Q4_1 streams; the "
                         "encoder forward of --config in --qtype")
    ap.add_argument("--encoder-steps", type=int, default=10, help="timed encodes of the encoder workload")
    ap.add_argument("--gemv-formats", default="Q8_0,Q4_0,Q4_1,Q5_0,Q5_1")
    ap.add_argument("--gemv-batches", default="1,5", help="GEMV microbench: batch sizes (up to 16)")
    ap.add_argument("--gemv-single", action="store_true",
                    help="GEMV microbench: single launches between event pairs only, no graph "
                         "(for kernel-trace profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench: the benchmark runs on one GPU; --gpus {args.gpus} is not supported "
              "(streams shard data-parallel across GPUs with no collective)", file=sys.stderr)
        sys.exit(2)
    if args.gemv:
        run_gemv(args)
    elif args.workload == "encoder":
        run_encoder(args)
    elif args.workload:
        run_batched(args)
    else:
        run_decode(args)


if __name__ == "__main__":
    main()
