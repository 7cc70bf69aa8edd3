"""Host-side mirror of the reference's decoder interface over libwhisper_hip.so.

The reference's decoder sits behind `model.Decoder`
(internal/model/interfaces.go:22-25):

    Decode(ctx, encoderOut ml.Tensor, params DecoderParams) ([]Segment, error)

`HIPDecoder.decode` has the same argument meaning and result: the encoder
output [T, n_state] float32, a `DecoderParams`, and a list with one `Segment`
holding every non-prompt token (internal/model/decoder.go:1415-1459; without an
attached vocabulary Text stays empty). Errors keep the reference's prefixes
("model: decoder: ...", "model: decode: ..."); shape errors raise
`ShapeMismatchError`, cancellation raises `CancelledError`.
"""
import ctypes as C
from dataclasses import dataclass, field
from typing import List, Optional, Sequence as Seq

import numpy as np

from . import native
from .native import check, lib


class ShapeMismatchError(ValueError):
    """ml.ErrShapeMismatch (internal/ml/tensor.go:6)."""


class CancelledError(RuntimeError):
    """context.Canceled observed between token steps."""


@dataclass
class DecoderParams:
    """model.DecoderParams (internal/model/interfaces.go:76-90)."""
    prompt: List[int] = field(default_factory=list)
    beam_size: int = 0
    best_of: int = 0
    temperature: float = 0.0
    temperature_inc: float = 0.0
    entropy_thold: float = 0.0
    logprob_thold: float = 0.0
    no_speech_thold: float = 0.0
    no_fallback: bool = False
    max_tokens: int = 0
    suppress_nst: bool = False
    suppress_regex: str = ""
    dtw_enabled: bool = False


@dataclass
class TokenData:
    """model.TokenData (internal/model/interfaces.go:57-67)."""
    id: int
    text: str = ""
    p: float = 0.0
    plog: float = 0.0
    pt: float = 0.0
    ptsum: float = 0.0
    t0: int = 0
    t1: int = 0
    tdtw: int = 0


@dataclass
class Segment:
    """model.Segment (internal/model/interfaces.go:47-54)."""
    start_ms: int = 0
    end_ms: int = 0
    text: str = ""
    tokens: List[TokenData] = field(default_factory=list)
    speaker: int = 0


def tokens_to_segments(tokens, prompt):
    """decoder.go:1415-1459 without a vocabulary: one segment with every
    non-prompt token (token texts are empty, so nothing is collapsed)."""
    if len(tokens) < len(prompt):
        return []
    rest = list(tokens[len(prompt):])
    if not rest:
        return []
    return [Segment(tokens=[TokenData(id=int(t)) for t in rest])]


def _params_struct(p: DecoderParams):
    prompt = (C.c_int32 * max(1, len(p.prompt)))(*[int(t) for t in p.prompt])
    s = native.WhDecodeParams(C.cast(prompt, C.POINTER(C.c_int32)), len(p.prompt), int(p.beam_size),
                              float(p.temperature), float(p.logprob_thold), float(p.no_speech_thold),
                              int(bool(p.no_fallback)), int(p.max_tokens), int(bool(p.suppress_nst)))
    return s, prompt


def _raise(rc):
    msg = lib().wh_last_error().decode(errors="replace")
    if rc == native.WH_ERR_CANCELLED:
        raise CancelledError(msg)
    if rc == native.WH_ERR_INVALID and "must be [T," in msg:
        raise ShapeMismatchError(msg)
    raise native.WhError(rc, msg)


def _tensor_table(tensors):
    arr = (native.WhTensor * len(tensors))()
    keep = []
    for i, t in enumerate(tensors):
        name = t.name.encode()
        keep.append(name)
        data = np.ascontiguousarray(t.data)
        keep.append(data)
        arr[i].name = name
        arr[i].type = t.type
        arr[i].ndim = len(t.shape)
        for j, s in enumerate(t.shape):
            arr[i].shape[j] = s
        arr[i].data = data.ctypes.data
        arr[i].nbytes = data.size
    return arr, keep


class HIPEncoder:
    """An encoder whose weights live in HBM (WhisperEncoder: NewEncoder + Encode,
    internal/model/encoder.go:58-338)."""

    def __init__(self, tensors=None, meta=None, device=0, gguf_path=None):
        h = C.c_void_p()
        if gguf_path is not None:
            rc = lib().wh_encoder_load_gguf(gguf_path.encode(), device, C.byref(h))
        else:
            arr, keep = _tensor_table(tensors)
            m = native.WhEncMeta(**(meta or {}))
            rc = lib().wh_encoder_create(arr, len(tensors), C.byref(m), device, C.byref(h))
            del keep
        if rc != native.WH_OK:
            _raise(rc)
        self._h = h
        hp = (C.c_int32 * 5)()
        check(lib().wh_encoder_hparams(h, hp))
        self.n_mels, self.n_state, self.n_head, self.n_layer, self.n_ctx = list(hp)

    @classmethod
    def from_gguf(cls, path, device=0):
        return cls(gguf_path=path, device=device)

    def close(self):
        if getattr(self, "_h", None):
            lib().wh_encoder_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def encode(self, mel, cancel: Optional[C.c_int32] = None):
        """mel [n_mels, T] float32 -> encoder output [T', n_state] (T' = (T + 1) / 2)."""
        mel = np.ascontiguousarray(mel, np.float32)
        if mel.ndim != 2:
            raise ShapeMismatchError(f"model: encoder: mel must be [{self.n_mels}, T], got {list(mel.shape)}")
        nm, t = mel.shape
        cap = (min(t, 2 * self.n_ctx) + 1) // 2
        out = np.empty((max(cap, 1), self.n_state), np.float32)
        rows = C.c_int32(0)
        cptr = C.cast(C.byref(cancel), C.c_void_p) if cancel is not None else None
        rc = lib().wh_encode(self._h, mel.ctypes.data, nm, t, out.ctypes.data, out.shape[0], C.byref(rows), cptr)
        if rc != native.WH_OK:
            _raise(rc)
        return out[:rows.value]

    def encode_device(self, mel_ptr, n_mels, T, out_ptr, out_cap, cancel: Optional[C.c_int32] = None):
        """Encode with mel ([n_mels, T] float32) and the output ([out_cap, n_state]
        float32) in device memory, given as addresses; returns the output rows."""
        rows = C.c_int32(0)
        cptr = C.cast(C.byref(cancel), C.c_void_p) if cancel is not None else None
        rc = lib().wh_encode_device(self._h, int(mel_ptr), n_mels, T, int(out_ptr), out_cap, C.byref(rows), cptr)
        if rc != native.WH_OK:
            _raise(rc)
        return rows.value


class HIPDecoder:
    """A decoder whose weights live in HBM (model.Decoder implementation)."""

    def __init__(self, tensors=None, meta=None, device=0, gguf_path=None):
        h = C.c_void_p()
        if gguf_path is not None:
            rc = lib().wh_model_load_gguf(gguf_path.encode(), device, C.byref(h))
        else:
            arr, keep = _tensor_table(tensors)
            m = native.WhMeta(**(meta or {}))
            rc = lib().wh_model_create(arr, len(tensors), C.byref(m), device, C.byref(h))
            del keep
        if rc != native.WH_OK:
            _raise(rc)
        self._h = h
        hp = (C.c_int32 * 5)()
        check(lib().wh_model_hparams(h, hp))
        self.n_vocab, self.n_state, self.n_head, self.n_layer, self.n_ctx = list(hp)
        self.eot = 50256

    @classmethod
    def from_gguf(cls, path, device=0):
        return cls(gguf_path=path, device=device)

    def close(self):
        if getattr(self, "_h", None):
            lib().wh_model_destroy(self._h)
            self._h = None

    __del__ = close

    def set_vocabulary(self, eot: Optional[int]):
        """SetVocabulary (decoder.go:85-94): only the EOT id is used on this path."""
        if eot is not None and eot >= 0:
            check(lib().wh_model_set_eot(self._h, int(eot)))
            self.eot = int(eot)

    def set_attention_mode(self, mode: int):
        check(lib().wh_model_set_attention_mode(self._h, int(mode)))

    @property
    def weight_bytes(self):
        b = C.c_uint64()
        check(lib().wh_model_weight_bytes(self._h, C.byref(b)))
        return b.value

    def _check_enc(self, enc):
        enc = np.ascontiguousarray(enc, dtype=np.float32)
        if enc.ndim != 2 or enc.shape[1] != self.n_state:
            raise ShapeMismatchError(
                f"model: decoder: encoder output must be [T, {self.n_state}], got {list(enc.shape)}")
        return enc

    def decode_tokens(self, encoder_out, params: DecoderParams, cancel: Optional[C.c_int32] = None):
        """Full token sequence (prompt + generated) of Decode."""
        enc = self._check_enc(encoder_out)
        ps, keep = _params_struct(params)
        # a beam history grows by at most one token per hypothesis and step (in-place reuse)
        cap = len(params.prompt) + max(1, int(params.beam_size)) * (self.n_ctx + 1) + 8
        out = (C.c_int32 * cap)()
        n = C.c_int32()
        cptr = C.pointer(cancel) if cancel is not None else None
        rc = lib().wh_decode(self._h, enc.ctypes.data, enc.shape[0], enc.shape[1], C.byref(ps), out, cap,
                             C.byref(n), cptr)
        if rc != native.WH_OK:
            _raise(rc)
        return list(out[:n.value])

    def decode_tokens_device(self, enc_ptr, enc_len, params: DecoderParams, cancel: Optional[C.c_int32] = None):
        """decode_tokens with the encoder output [enc_len, n_state] float32 in device
        memory of the model's device, given as an address."""
        ps, keep = _params_struct(params)
        cap = len(params.prompt) + max(1, int(params.beam_size)) * (self.n_ctx + 1) + 8
        out = (C.c_int32 * cap)()
        n = C.c_int32()
        cptr = C.pointer(cancel) if cancel is not None else None
        rc = lib().wh_decode_device(self._h, int(enc_ptr), int(enc_len), self.n_state, C.byref(ps), out, cap,
                                    C.byref(n), cptr)
        if rc != native.WH_OK:
            _raise(rc)
        return list(out[:n.value])

    @staticmethod
    def last_decode_steps():
        """Forward steps of this thread's last decode_tokens / decode / decode_batch
        call (a beam hypothesis may grow by more than one token per step)."""
        n = C.c_int32(0)
        check(lib().wh_last_decode_steps(C.byref(n)))
        return n.value

    def decode(self, encoder_out, params: DecoderParams, cancel=None) -> List[Segment]:
        """(*WhisperDecoder).Decode (internal/model/decoder.go:401-410)."""
        return tokens_to_segments(self.decode_tokens(encoder_out, params, cancel), params.prompt)

    def decode_batch(self, encoder_outs: Seq[np.ndarray], params: Seq[DecoderParams], cancel=None):
        """Greedy decode of independent streams as one batch; token lists per stream."""
        S = len(encoder_outs)
        encs = [self._check_enc(e) for e in encoder_outs]
        if len({e.shape[0] for e in encs}) != 1:
            raise ShapeMismatchError("model: decoder: batched streams need equal encoder lengths")
        ptrs = (C.c_void_p * S)(*[e.ctypes.data for e in encs])
        structs, keep = [], []
        for p in params:
            s, k = _params_struct(p)
            structs.append(s)
            keep.append(k)
        parr = (native.WhDecodeParams * S)(*structs)
        cap = max(len(p.prompt) for p in params) + self.n_ctx + 8
        out = (C.c_int32 * (S * cap))()
        lens = (C.c_int32 * S)()
        cptr = C.pointer(cancel) if cancel is not None else None
        rc = lib().wh_decode_batch(self._h, S, ptrs, encs[0].shape[0], self.n_state, parr, out, cap, lens, cptr)
        if rc != native.WH_OK:
            _raise(rc)
        return [list(out[i * cap:i * cap + lens[i]]) for i in range(S)]

    def sequence(self, encoder_outs, shared_encoder=False):
        return Sequence(self, encoder_outs, shared_encoder)


class Sequence:
    """Step-level decoder states (decoderState, decoder.go:306-386) for S streams."""

    def __init__(self, dec: HIPDecoder, encoder_outs, shared_encoder=False):
        self.dec = dec
        encs = [dec._check_enc(e) for e in encoder_outs]
        self.S = len(encs)
        ptrs = (C.c_void_p * self.S)(*[e.ctypes.data for e in encs])
        h = C.c_void_p()
        rc = lib().wh_seq_create(dec._h, self.S, ptrs, encs[0].shape[0], dec.n_state, int(bool(shared_encoder)),
                                 C.byref(h))
        if rc != native.WH_OK:
            _raise(rc)
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            lib().wh_seq_destroy(self._h)
            self._h = None

    __del__ = close

    def set_tokens(self, stream, tokens, reset_kv=False):
        arr = (C.c_int32 * max(1, len(tokens)))(*[int(t) for t in tokens])
        rc = lib().wh_seq_set_tokens(self._h, stream, arr, len(tokens), int(bool(reset_kv)))
        if rc != native.WH_OK:
            _raise(rc)

    def _active(self, active):
        if active is None:
            return None
        return (C.c_int32 * self.S)(*[int(bool(a)) for a in active])

    def step_greedy(self, active=None, temperature=1.0, suppress_nst=False, no_speech_thold=0.0, logits=False):
        ids = (C.c_int32 * self.S)()
        out = np.empty((self.S, self.dec.n_vocab), np.float32) if logits else None
        rc = lib().wh_seq_step_greedy(self._h, self._active(active), float(temperature), int(bool(suppress_nst)),
                                      float(no_speech_thold), ids, out.ctypes.data if logits else None)
        if rc != native.WH_OK:
            _raise(rc)
        return (list(ids), out) if logits else list(ids)

    def generate(self, n, temperature=1.0, suppress_nst=False, no_speech_thold=0.0, max_len=None):
        """Up to n greedy steps of stream 0 with the reference's stop rules."""
        ids = (C.c_int32 * max(1, n))()
        got = C.c_int32()
        ml = self.dec.n_ctx if max_len is None else int(max_len)
        rc = lib().wh_seq_generate(self._h, int(n), float(temperature), int(bool(suppress_nst)),
                                   float(no_speech_thold), ml, ids, C.byref(got))
        if rc != native.WH_OK:
            _raise(rc)
        return list(ids[:got.value])

    @property
    def persistent(self):
        """(served by the persistent kernel, persistent launches so far)."""
        on, n = C.c_int32(), C.c_int64()
        check(lib().wh_seq_persistent(self._h, C.byref(on), C.byref(n)))
        return bool(on.value), n.value

    def set_profiling(self, enable):
        check(lib().wh_seq_set_profiling(self._h, int(bool(enable))))

    def profile(self):
        """{kernel class: (ms, launches, algorithmic bytes)} accumulated since
        profiling was enabled."""
        n = C.c_int32()
        check(lib().wh_seq_profile_count(self._h, C.byref(n)))
        out = {}
        for i in range(n.value):
            name = C.create_string_buffer(64)
            ms, cnt, by = C.c_double(), C.c_int64(), C.c_double()
            check(lib().wh_seq_profile_get(self._h, i, name, 64, C.byref(ms), C.byref(cnt), C.byref(by)))
            out[name.value.decode()] = (ms.value, cnt.value, by.value)
        return out

    def step_topk(self, k=5, active=None, temperature=1.0, logits=False):
        tok = (C.c_int32 * (self.S * k))()
        lp = (C.c_float * (self.S * k))()
        out = np.empty((self.S, self.dec.n_vocab), np.float32) if logits else None
        rc = lib().wh_seq_step_topk(self._h, self._active(active), k, float(temperature), tok, lp,
                                    out.ctypes.data if logits else None)
        if rc != native.WH_OK:
            _raise(rc)
        t = np.array(tok[:], np.int32).reshape(self.S, k)
        l = np.array(lp[:], np.float32).reshape(self.S, k)
        return (t, l, out) if logits else (t, l)
