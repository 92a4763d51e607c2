"""MI355X (gfx950) integer I-Whisper encoder/decoder path.

Layer API mirroring the reference's i_whisper/model_int.py and
i_whisper/modules/linear.py, backed by hand-written HIP kernels reached through
the C ABI in include/iwhisper_amd.h.
"""
from . import _lib, kernels  # noqa: F401
