"""ctypes bindings of libwhisper_hip.so (declarations: include/whisper_hip.h).

The library is loaded from whisper.go_amd/lib/ only; a missing library is an
error (there is no fallback implementation).
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libwhisper_hip.so")

WH_OK = 0
WH_ERR_INVALID = -1
WH_ERR_HIP = -2
WH_ERR_UNSUPPORTED = -3
WH_ERR_CANCELLED = -4
WH_ERR_NOMEM = -5
WH_ERR_NOT_FOUND = -6

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q5_0, TYPE_Q5_1, TYPE_Q8_0 = 0, 1, 2, 3, 6, 7, 8
TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0"}
TYPE_CODES = {v: k for k, v in TYPE_NAMES.items()}


class WhTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("ndim", C.c_uint32),
                ("shape", C.c_uint64 * 4), ("data", C.c_void_p), ("nbytes", C.c_uint64)]


class WhMeta(C.Structure):
    _fields_ = [("n_head", C.c_uint32), ("n_layer", C.c_uint32), ("n_ctx", C.c_uint32),
                ("n_state", C.c_uint32), ("n_vocab", C.c_uint32)]


class WhEncMeta(C.Structure):
    _fields_ = [("n_head", C.c_uint32), ("n_layer", C.c_uint32), ("n_ctx", C.c_uint32),
                ("n_state", C.c_uint32), ("n_mels", C.c_uint32)]


class WhDecodeParams(C.Structure):
    _fields_ = [("prompt", C.POINTER(C.c_int32)), ("prompt_len", C.c_int32), ("beam_size", C.c_int32),
                ("temperature", C.c_float), ("logprob_thold", C.c_float), ("no_speech_thold", C.c_float),
                ("no_fallback", C.c_int32), ("max_tokens", C.c_int32), ("suppress_nst", C.c_int32)]


class WhError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{msg} (status {code})")
        self.code = code


# (name, restype, argtypes) of every exported entry point
_P = C.c_void_p
_SIGS = [
    ("wh_last_error", C.c_char_p, []),
    ("wh_version", C.c_char_p, []),
    ("wh_device_count", C.c_int, [C.POINTER(C.c_int32)]),
    ("wh_dev_malloc", C.c_int, [C.c_uint64, C.c_int32, C.POINTER(_P)]),
    ("wh_dev_free", C.c_int, [_P]),
    ("wh_memcpy", C.c_int, [_P, _P, C.c_uint64, C.c_int32]),
    ("wh_stream_create", C.c_int, [C.c_int32, C.POINTER(_P)]),
    ("wh_stream_destroy", C.c_int, [_P]),
    ("wh_stream_sync", C.c_int, [_P]),
    ("wh_event_create", C.c_int, [C.POINTER(_P)]),
    ("wh_event_destroy", C.c_int, [_P]),
    ("wh_event_record", C.c_int, [_P, _P]),
    ("wh_event_elapsed", C.c_int, [_P, _P, C.POINTER(C.c_float)]),
    ("wh_row_bytes", C.c_uint64, [C.c_uint32, C.c_uint64]),
    ("wh_quantize", C.c_int, [C.c_uint32, _P, C.c_uint64, _P, C.c_uint64, C.c_int32]),
    ("wh_should_quantize", C.c_int, [C.c_char_p]),
    ("wh_f32_to_f16", C.c_uint16, [C.c_float]),
    ("wh_f16_to_f32", C.c_float, [C.c_uint16]),
    ("wh_dequantize", C.c_int, [C.c_uint32, _P, C.c_uint64, C.c_uint64, _P, C.c_int32]),
    ("wh_dequantize_noalloc", C.c_int, [C.c_uint32, _P, C.c_uint64, C.c_uint64, _P, C.c_int32]),
    ("wh_last_decode_steps", C.c_int, [C.POINTER(C.c_int32)]),
    ("wh_matrix_create", C.c_int, [C.c_uint32, C.c_int32, C.c_int32, _P, C.c_uint64, C.c_int32, C.POINTER(_P)]),
    ("wh_matrix_destroy", C.c_int, [_P]),
    ("wh_matrix_bytes", C.c_int, [_P, C.POINTER(C.c_uint64)]),
    ("wh_gemv", C.c_int, [_P, _P, C.c_int32, _P, _P]),
    ("wh_model_create", C.c_int, [C.POINTER(WhTensor), C.c_int32, C.POINTER(WhMeta), C.c_int32, C.POINTER(_P)]),
    ("wh_model_load_gguf", C.c_int, [C.c_char_p, C.c_int32, C.POINTER(_P)]),
    ("wh_encoder_create", C.c_int, [C.POINTER(WhTensor), C.c_int32, C.POINTER(WhEncMeta), C.c_int32, C.POINTER(_P)]),
    ("wh_encoder_load_gguf", C.c_int, [C.c_char_p, C.c_int32, C.POINTER(_P)]),
    ("wh_encoder_destroy", C.c_int, [_P]),
    ("wh_encoder_hparams", C.c_int, [_P, C.POINTER(C.c_int32)]),
    ("wh_encode", C.c_int, [_P, _P, C.c_int32, C.c_int32, _P, C.c_int32, C.POINTER(C.c_int32), _P]),
    ("wh_encode_device", C.c_int, [_P, _P, C.c_int32, C.c_int32, _P, C.c_int32, C.POINTER(C.c_int32), _P]),
    ("wh_model_destroy", C.c_int, [_P]),
    ("wh_model_hparams", C.c_int, [_P, C.POINTER(C.c_int32)]),
    ("wh_model_set_eot", C.c_int, [_P, C.c_int32]),
    ("wh_model_weight_bytes", C.c_int, [_P, C.POINTER(C.c_uint64)]),
    ("wh_model_set_attention_mode", C.c_int, [_P, C.c_int32]),
    ("wh_decode", C.c_int, [_P, _P, C.c_int32, C.c_int32, C.POINTER(WhDecodeParams), C.POINTER(C.c_int32),
                            C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    ("wh_decode_device", C.c_int, [_P, _P, C.c_int32, C.c_int32, C.POINTER(WhDecodeParams), C.POINTER(C.c_int32),
                            C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    ("wh_decode_batch", C.c_int, [_P, C.c_int32, C.POINTER(_P), C.c_int32, C.c_int32, C.POINTER(WhDecodeParams),
                                  C.POINTER(C.c_int32), C.c_int32, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    ("wh_seq_create", C.c_int, [_P, C.c_int32, C.POINTER(_P), C.c_int32, C.c_int32, C.c_int32, C.POINTER(_P)]),
    ("wh_seq_create_device", C.c_int, [_P, C.c_int32, C.POINTER(_P), C.c_int32, C.c_int32, C.c_int32, C.POINTER(_P)]),
    ("wh_seq_destroy", C.c_int, [_P]),
    ("wh_seq_set_tokens", C.c_int, [_P, C.c_int32, C.POINTER(C.c_int32), C.c_int32, C.c_int32]),
    ("wh_seq_step_greedy", C.c_int, [_P, C.POINTER(C.c_int32), C.c_float, C.c_int32, C.c_float,
                                     C.POINTER(C.c_int32), _P]),
    ("wh_seq_step_topk", C.c_int, [_P, C.POINTER(C.c_int32), C.c_int32, C.c_float, C.POINTER(C.c_int32),
                                   C.POINTER(C.c_float), _P]),
    ("wh_seq_generate", C.c_int, [_P, C.c_int32, C.c_float, C.c_int32, C.c_float, C.c_int32,
                                  C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    ("wh_seq_persistent", C.c_int, [_P, C.POINTER(C.c_int32), C.POINTER(C.c_int64)]),
    ("wh_seq_set_profiling", C.c_int, [_P, C.c_int32]),
    ("wh_seq_profile_count", C.c_int, [_P, C.POINTER(C.c_int32)]),
    ("wh_seq_profile_get", C.c_int, [_P, C.c_int32, C.c_char_p, C.c_int32, C.POINTER(C.c_double),
                                     C.POINTER(C.c_int64), C.POINTER(C.c_double)]),
]
EXPORTED = [s[0] for s in _SIGS]

_lib = None


def lib():
    """Load libwhisper_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing: build it with `python whisper.go_amd/build.py`")
        L = C.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != WH_OK:
        raise WhError(rc, lib().wh_last_error().decode(errors="replace"))
    return rc


def device_count():
    n = C.c_int32(0)
    check(lib().wh_device_count(C.byref(n)))
    return n.value


class DevBuf:
    """A device allocation owned by the library's HIP runtime."""

    def __init__(self, nbytes, device=0):
        self.ptr = C.c_void_p()
        self.nbytes = int(nbytes)
        check(lib().wh_dev_malloc(self.nbytes, device, C.byref(self.ptr)))

    @classmethod
    def from_array(cls, a, device=0):
        import numpy as np

        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, device)
        b.upload(a)
        return b

    def upload(self, a):
        import numpy as np

        a = np.ascontiguousarray(a)
        check(lib().wh_memcpy(self.ptr, a.ctypes.data, a.nbytes, 0))

    def download(self, shape, dtype):
        import numpy as np

        out = np.empty(shape, dtype)
        check(lib().wh_memcpy(out.ctypes.data, self.ptr, out.nbytes, 1))
        return out

    def free(self):
        if self.ptr:
            lib().wh_dev_free(self.ptr)
            self.ptr = C.c_void_p()

    __del__ = free


class Stream:
    def __init__(self, device=0):
        self.h = C.c_void_p()
        check(lib().wh_stream_create(device, C.byref(self.h)))

    def sync(self):
        check(lib().wh_stream_sync(self.h))

    def close(self):
        if self.h:
            lib().wh_stream_destroy(self.h)
            self.h = C.c_void_p()

    __del__ = close


class Event:
    def __init__(self):
        self.h = C.c_void_p()
        check(lib().wh_event_create(C.byref(self.h)))

    def record(self, stream):
        check(lib().wh_event_record(self.h, stream.h if isinstance(stream, Stream) else stream))

    def elapsed_ms(self, later):
        ms = C.c_float()
        check(lib().wh_event_elapsed(self.h, later.h, C.byref(ms)))
        return ms.value

    def close(self):
        if self.h:
            lib().wh_event_destroy(self.h)
            self.h = C.c_void_p()

    __del__ = close
