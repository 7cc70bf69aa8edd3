"""MI355X (gfx950) decoder token loop for whisper.go.

The compute path is libwhisper_hip.so (hand-written HIP kernels, C ABI in
include/whisper_hip.h); this package is the host-side mirror of the
reference's decoder interface plus fixture tooling. Import it by path (the
directory name contains a dot), e.g. via __graft_entry__.load_package().
"""
from . import native, quant, synth  # noqa: F401
from .model import (CancelledError, DecoderParams, HIPDecoder, HIPEncoder, Segment, Sequence,  # noqa: F401
                    ShapeMismatchError, TokenData, tokens_to_segments)

__all__ = ["native", "quant", "synth", "HIPDecoder", "HIPEncoder", "Sequence", "DecoderParams", "Segment", "TokenData",
           "ShapeMismatchError", "CancelledError", "tokens_to_segments"]
