"""Seeded synthetic whisper decoders in the reference's tensor names and shapes,
quantised by the reference's `cmd/quantize` rule, plus GGUF v3 writing/reading.

* Tensor naming and shapes follow internal/model/decoder.go:176-296 (rows
  first, as stored in GGUF descriptors).
* Quantisation follows gguf.QuantizeFile (internal/gguf/quantize.go:50-117):
  tensors for which shouldQuantize(name) holds (internal/gguf/quant.go:236-248)
  are quantised flat to the target type, the rest stay F32. This quantises the
  token embedding and the per-block LN gains (names contain "_ln." not ".ln").
* Values: matrices, embeddings, biases, LN biases and positional embedding
  ~ N(0, 0.02); LN gains 1 + N(0, 0.02). Each tensor draws from its own
  PCG64 stream seeded by a hash of "<config>/<tensor name>".
* The GGUF writer follows internal/gguf/writer.go:24-107 (v3, 32-byte aligned).
"""
import hashlib
import struct

import numpy as np

from . import quant

CONFIGS = {
    # name: (n_vocab, n_state, n_head, n_layer, n_ctx)
    "tiny.en": (51864, 384, 6, 4, 448),
    "base": (51865, 512, 8, 6, 448),
    "small": (51864, 768, 12, 12, 448),
    "medium": (51865, 1024, 16, 24, 448),
    "large-v3": (51866, 1280, 20, 32, 448),
}
ENC_LEN = 1500
SOT_EN_TRANSCRIBE = [50258, 50259, 50359]  # buildPrompt with models/tokenizer.json ids


def seed_of(config, name):
    return int.from_bytes(hashlib.sha256(f"{config}/{name}".encode()).digest()[:8], "little")


def rng_for(config, name):
    return np.random.Generator(np.random.PCG64(seed_of(config, name)))


def tensor_specs(n_vocab, d, n_layer, n_ctx):
    """(name, shape) of every decoder tensor, in the reference's load order."""
    specs = [("decoder.token_embedding.weight", (n_vocab, d)), ("decoder.positional_embedding", (n_ctx, d))]
    for i in range(n_layer):
        p = f"decoder.blocks.{i}."
        for sub in ("self_attn", "cross_attn"):
            specs += [(p + f"{sub}_ln.weight", (d,)), (p + f"{sub}_ln.bias", (d,)),
                      (p + f"{sub}.query.weight", (d, d)), (p + f"{sub}.query.bias", (d,)),
                      (p + f"{sub}.key.weight", (d, d)),
                      (p + f"{sub}.value.weight", (d, d)), (p + f"{sub}.value.bias", (d,)),
                      (p + f"{sub}.out.weight", (d, d)), (p + f"{sub}.out.bias", (d,))]
        specs += [(p + "mlp_ln.weight", (d,)), (p + "mlp_ln.bias", (d,)),
                  (p + "mlp.0.weight", (4 * d, d)), (p + "mlp.0.bias", (4 * d,)),
                  (p + "mlp.2.weight", (d, 4 * d)), (p + "mlp.2.bias", (d,))]
    specs += [("decoder.ln.weight", (d,)), ("decoder.ln.bias", (d,))]
    return specs


def is_ln_gain(name):
    return name.endswith("_ln.weight") or name in ("decoder.ln.weight", "encoder.ln_post.weight")


def gen_f32(config, name, shape, std=0.02):
    n = int(np.prod(shape))
    x = rng_for(config, name).standard_normal(n, dtype=np.float32)
    x *= np.float32(std)
    if is_ln_gain(name):
        x += np.float32(1.0)
    return x.reshape(shape)


class Tensor:
    """One GGUF tensor: name, type code, shape (rows first), raw bytes."""
    __slots__ = ("name", "type", "shape", "data")

    def __init__(self, name, qtype, shape, data):
        self.name, self.type, self.shape = name, int(qtype), tuple(int(s) for s in shape)
        self.data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)

    def __repr__(self):
        return f"Tensor({self.name!r}, type={self.type}, shape={self.shape}, {self.data.size} B)"


def make_decoder(config="tiny.en", qtype=8, dims=None, std=0.02):
    """Synthetic decoder tensors quantised with the cmd/quantize rule.

    dims overrides CONFIGS[config] with (n_vocab, n_state, n_head, n_layer, n_ctx).
    Returns (tensors, meta) where meta holds the whisper.decoder.* values.
    """
    V, d, H, L, ctx = dims if dims is not None else CONFIGS[config]
    out = []
    for name, shape in tensor_specs(V, d, L, ctx):
        x = gen_f32(config, name, shape, std)
        if qtype != 0 and quant.should_quantize(name):
            out.append(Tensor(name, qtype, shape, quant.quantize(qtype, x)))
        else:
            out.append(Tensor(name, 0, shape, x))
    meta = dict(n_head=H, n_layer=L, n_ctx=ctx, n_state=d, n_vocab=V)
    return out, meta


# encoder: (n_mels, n_state, n_head, n_layer, n_audio_ctx)
ENC_CONFIGS = {
    "tiny.en": (80, 384, 6, 4, 1500),
    "base": (80, 512, 8, 6, 1500),
    "small": (80, 768, 12, 12, 1500),
    "medium": (80, 1024, 16, 24, 1500),
    "large-v3": (128, 1280, 20, 32, 1500),
}


def encoder_specs(n_mels, d, n_layer, n_ctx):
    """(name, shape) of every encoder tensor (internal/model/encoder.go:58-263)."""
    specs = [("encoder.conv1.weight", (d, n_mels, 3)), ("encoder.conv1.bias", (d,)),
             ("encoder.conv2.weight", (d, d, 3)), ("encoder.conv2.bias", (d,)),
             ("encoder.positional_embedding", (n_ctx, d))]
    for i in range(n_layer):
        p = f"encoder.blocks.{i}."
        specs += [(p + "attn_ln.weight", (d,)), (p + "attn_ln.bias", (d,)),
                  (p + "attn.query.weight", (d, d)), (p + "attn.query.bias", (d,)),
                  (p + "attn.key.weight", (d, d)),
                  (p + "attn.value.weight", (d, d)), (p + "attn.value.bias", (d,)),
                  (p + "attn.out.weight", (d, d)), (p + "attn.out.bias", (d,)),
                  (p + "mlp_ln.weight", (d,)), (p + "mlp_ln.bias", (d,)),
                  (p + "mlp.0.weight", (4 * d, d)), (p + "mlp.0.bias", (4 * d,)),
                  (p + "mlp.2.weight", (d, 4 * d)), (p + "mlp.2.bias", (d,))]
    specs += [("encoder.ln_post.weight", (d,)), ("encoder.ln_post.bias", (d,))]
    return specs


def make_encoder(config="tiny.en", qtype=8, dims=None, std=0.02):
    """Synthetic encoder tensors quantised with the cmd/quantize rule (the conv
    weights and the block LN gains too, as the rule quantises every ".weight"
    whose name has neither "norm" nor ".ln"). dims overrides ENC_CONFIGS[config]
    with (n_mels, n_state, n_head, n_layer, n_audio_ctx). Returns (tensors, meta)."""
    M, d, H, L, ctx = dims if dims is not None else ENC_CONFIGS[config]
    out = []
    for name, shape in encoder_specs(M, d, L, ctx):
        x = gen_f32(config, name, shape, std)
        if qtype != 0 and quant.should_quantize(name) and x.size % 32 == 0:
            out.append(Tensor(name, qtype, shape, quant.quantize(qtype, x)))
        else:
            out.append(Tensor(name, 0, shape, x))
    meta = dict(n_head=H, n_layer=L, n_ctx=ctx, n_state=d, n_mels=M)
    return out, meta


def mel_input(config, n_mels, T=3000, stream=0):
    """Synthetic log-mel input [n_mels, T] ~ N(0, 0.5), seeded per stream."""
    return (0.5 * rng_for(config, f"mel/{stream}").standard_normal((n_mels, T))).astype(np.float32)


def stream_prompts(n_streams=16, seed=16, min_len=4, max_len=224):
    """Prompts of the multi-stream workload: SOT/en/transcribe followed by ids
    drawn from [0, 50000), total lengths uniform in [min_len, max_len]."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(min_len, max_len + 1, size=n_streams)
    ids = rng.integers(0, 50000, size=(n_streams, max_len))
    return [SOT_EN_TRANSCRIBE + [int(t) for t in ids[i, :lens[i] - len(SOT_EN_TRANSCRIBE)]]
            for i in range(n_streams)]


def encoder_output(config, d, stream=0, enc_len=ENC_LEN):
    """Synthetic encoder output [enc_len, d] ~ N(0, 1), seeded per stream."""
    return rng_for(config, f"encoder/{stream}").standard_normal((enc_len, d), dtype=np.float32)


def reference_test_decoder():
    """The reference's hand-built decoder fixture (internal/model/decoder_test.go:22-86):
    d=4, 2 heads, 1 layer, V=51865, ctx 128, every weight 0.01, LN gains 1,
    biases 0 — stored as F32 tensors."""
    V, d, H, L, ctx = 51865, 4, 2, 1, 128
    out = []
    for name, shape in tensor_specs(V, d, L, ctx):
        if is_ln_gain(name):
            x = np.ones(shape, np.float32)
        elif name.endswith(".bias"):
            x = np.zeros(shape, np.float32)
        else:
            x = np.full(shape, 0.01, np.float32)
        out.append(Tensor(name, 0, shape, x))
    return out, dict(n_head=H, n_layer=L, n_ctx=ctx, n_state=d, n_vocab=V)


def weight_bytes_per_token(tensors):
    """Quantised-weight bytes read per token: 14 d^2 per layer (self q/k/v/o,
    cross q/o, fc1, fc2) plus the tied logits matrix."""
    per = {t.name: t.data.size for t in tensors}
    total = per["decoder.token_embedding.weight"]
    for name, nbytes in per.items():
        if not name.startswith("decoder.blocks.") or not name.endswith(".weight"):
            continue
        if any(s in name for s in ("_ln.", "cross_attn.key", "cross_attn.value")):
            continue
        total += nbytes
    return total


# ---- GGUF v3 ------------------------------------------------------------------
GGUF_MAGIC = 0x46554747


def _gstr(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


_META_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


def write_gguf(path, tensors, meta=None, extra=None):
    """Write tensors (+ uint32 whisper.* metadata) as GGUF v3
    (internal/gguf/writer.go:24-107: 32-byte aligned header and tensors).
    extra: further metadata as (key, gguf type code, value); type 8 is a string,
    type 9 an array given as (element type, [values])."""
    kv = []
    keys = {"n_head": "whisper.decoder.attention.head_count", "n_layer": "whisper.decoder.layer_count",
            "n_ctx": "whisper.decoder.context_length", "n_state": "whisper.decoder.embedding_length",
            "n_vocab": "whisper.vocab.size"}
    for k, v in (meta or {}).items():
        kv.append(_gstr(keys[k]) + struct.pack("<II", 4, int(v)))

    def value(t, v):
        if t == 8:
            return _gstr(v)
        if t == 9:
            et, vals = v
            return struct.pack("<IQ", et, len(vals)) + b"".join(value(et, x) for x in vals)
        return struct.pack(_META_FMT[t], v)

    for k, t, v in (extra or []):
        kv.append(_gstr(k) + struct.pack("<I", t) + value(t, v))
    infos, offsets, off = [], [], 0
    for t in tensors:
        offsets.append(off)
        off += t.data.size
        if off % 32:
            off += 32 - off % 32
    for t, o in zip(tensors, offsets):
        infos.append(_gstr(t.name) + struct.pack("<I", len(t.shape)) +
                     b"".join(struct.pack("<Q", s) for s in t.shape) + struct.pack("<IQ", t.type, o))
    header = struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(kv)) + b"".join(kv) + b"".join(infos)
    pad = (32 - len(header) % 32) % 32
    with open(path, "wb") as f:
        f.write(header + b"\0" * pad)
        for i, t in enumerate(tensors):
            f.write(t.data.tobytes())
            if i < len(tensors) - 1 and t.data.size % 32:
                f.write(b"\0" * (32 - t.data.size % 32))


def read_gguf(path):
    """Parse a GGUF v2/v3 file written by write_gguf (uint32 metadata only)."""
    buf = open(path, "rb").read()
    magic, version, nt, nm = struct.unpack_from("<IIQQ", buf, 0)
    if magic != GGUF_MAGIC or version not in (2, 3):
        raise ValueError("gguf: invalid magic or version")
    p = 24
    meta = {}

    def rstr(p):
        (n,) = struct.unpack_from("<Q", buf, p)
        return buf[p + 8:p + 8 + n].decode(), p + 8 + n

    for _ in range(nm):
        k, p = rstr(p)
        (vt,) = struct.unpack_from("<I", buf, p)
        p += 4
        if vt != 4:
            raise ValueError("read_gguf: only uint32 metadata is supported")
        (meta[k],) = struct.unpack_from("<I", buf, p)
        p += 4
    descs = []
    for _ in range(nt):
        name, p = rstr(p)
        (nd,) = struct.unpack_from("<I", buf, p)
        shape = struct.unpack_from("<" + "Q" * nd, buf, p + 4)
        qtype, off = struct.unpack_from("<IQ", buf, p + 4 + 8 * nd)
        p += 4 + 8 * nd + 12
        descs.append((name, qtype, shape, off))
    align = meta.get("general.alignment", 32)
    start = (p + align - 1) // align * align
    out = []
    for name, qtype, shape, off in descs:
        n = int(np.prod(shape))
        nb = n * 4 if qtype == 0 else n * 2 if qtype == 1 else (n + 31) // 32 * quant.BLOCK_BYTES[qtype]
        out.append(Tensor(name, qtype, shape, np.frombuffer(buf, np.uint8, nb, start + off)))
    return out, meta
