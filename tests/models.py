"""Synthetic decoders with hand-controlled logits, shared by the CPU and GPU tests."""
import numpy as np


def forced_repeat_model(wh, T, qtype=8, dims=(600, 64, 2, 1, 64), name="repeat", gap=100.0):
    """A decoder whose logits do not depend on its input: the final LayerNorm
    has gain 0, so its output is its bias beta, and the tied logits are
    E[t] . beta. Row T of the embedding is gap * beta / |beta|^2, so token T's
    logit is `gap` and every other is O(0.1). Quantised by the cmd/quantize rule."""
    d = dims[1]
    tensors, meta = wh.synth.make_decoder(name, 0, dims=dims)
    beta = wh.synth.rng_for(name, "beta").standard_normal(d).astype(np.float32)
    out = []
    for t in tensors:
        x = t.data.view(np.float32).reshape(t.shape).copy()
        if t.name == "decoder.ln.weight":
            x[:] = 0
        elif t.name == "decoder.ln.bias":
            x[:] = beta
        elif t.name == "decoder.token_embedding.weight":
            x[T] = np.float32(gap) * beta / np.float32(beta @ beta)
        if qtype and wh.quant.should_quantize(t.name):
            out.append(wh.synth.Tensor(t.name, qtype, t.shape, wh.quant.quantize(qtype, x)))
        else:
            out.append(wh.synth.Tensor(t.name, 0, t.shape, x))
    return out, meta
